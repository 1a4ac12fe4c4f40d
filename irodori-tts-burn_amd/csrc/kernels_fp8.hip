// fp8 (e4m3fn) GEMM operands for the fp8 compute mode (no counterpart in the reference,
// whose backends compute in f32 / f16 / bf16):
//   * weights: per output channel n (a row of the K-major matrix), s_n = max_k |w| / 448
//     and codes e4m3(w / s_n) (round to nearest even);
//   * activations (a GEMM's A operand): per row and 32-wide k block the power of two 2^e
//     with e the smallest integer such that max |x| <= 448 * 2^e, codes e4m3(x * 2^-e),
//     and the E8M0 byte 127 + e, the block-scale operand of the gfx950 scaled MFMA.
// The scales never let a code exceed 448, so the hardware converter (round to nearest
// even; it yields NaN past the e4m3 range) is exact here.
#include "common.hpp"
#include "kernels.hpp"

namespace irodori {

namespace {

// One 256-thread block per output channel: the channel's scale, then its codes.
__global__ __launch_bounds__(256) void quant_weight_rows_kernel(const float* __restrict__ w, int K,
                                                                uint8_t* __restrict__ q, float* __restrict__ s) {
    __shared__ float red[4];
    const int n = blockIdx.x, tid = threadIdx.x;
    const float* wr = w + (size_t)n * K;
    float amax = 0.f;
    for (int k = tid; k < K; k += 256) amax = fmaxf(amax, fabsf(wr[k]));
    for (int off = 32; off > 0; off >>= 1) amax = fmaxf(amax, __shfl_xor(amax, off));
    if ((tid & 63) == 0) red[tid >> 6] = amax;
    __syncthreads();
    amax = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    const float sn = amax > 0.f ? __fdiv_rn(amax, 448.f) : 1.f;
    if (tid == 0) s[n] = sn;
    for (int k4 = tid; k4 < K / 4; k4 += 256) {
        const float4 v = *reinterpret_cast<const float4*>(wr + 4 * k4);
        *reinterpret_cast<unsigned*>(q + (size_t)n * K + 4 * k4) =
            pack_e4m3(__fdiv_rn(v.x, sn), __fdiv_rn(v.y, sn), __fdiv_rn(v.z, sn), __fdiv_rn(v.w, sn));
    }
}

// One thread per 32-wide block of a row: 32 codes and the block's E8M0 byte.
template <typename T>
__global__ __launch_bounds__(256) void mx_quant_rows_kernel(const T* __restrict__ x, long nblocks,
                                                            uint8_t* __restrict__ q, uint8_t* __restrict__ s) {
    const long b = (long)blockIdx.x * 256 + threadIdx.x;
    if (b >= nblocks) return;
    const T* xb = x + b * 32;
    float v[32];
    if constexpr (sizeof(T) == 2) {
#pragma unroll
        for (int c = 0; c < 4; c++) {
            const bf16x8 h = *reinterpret_cast<const bf16x8*>(xb + 8 * c);
#pragma unroll
            for (int i = 0; i < 8; i++) v[8 * c + i] = static_cast<float>(h[i]);
        }
    } else {
#pragma unroll
        for (int c = 0; c < 8; c++) {
            const float4 f = *reinterpret_cast<const float4*>(xb + 4 * c);
            v[4 * c] = f.x; v[4 * c + 1] = f.y; v[4 * c + 2] = f.z; v[4 * c + 3] = f.w;
        }
    }
    float amax = 0.f;
#pragma unroll
    for (int i = 0; i < 32; i++) amax = fmaxf(amax, fabsf(v[i]));
    const int e = mx_exp(amax);
    s[b] = (uint8_t)(127 + e);
    unsigned w[8];
#pragma unroll
    for (int i = 0; i < 8; i++)
        w[i] = pack_e4m3(ldexpf(v[4 * i], -e), ldexpf(v[4 * i + 1], -e), ldexpf(v[4 * i + 2], -e),
                         ldexpf(v[4 * i + 3], -e));
    uint4* qo = reinterpret_cast<uint4*>(q + b * 32);
    qo[0] = make_uint4(w[0], w[1], w[2], w[3]);
    qo[1] = make_uint4(w[4], w[5], w[6], w[7]);
}

}  // namespace

void launch_quant_weight_rows(const float* w, int N, int K, uint8_t* q, float* s, hipStream_t st) {
    quant_weight_rows_kernel<<<N, 256, 0, st>>>(w, K, q, s);
}

template <typename T>
void launch_mx_quant_rows(const T* x, int M, int K, uint8_t* q, uint8_t* s, hipStream_t st) {
    const long nb = (long)M * (K / 32);
    if (nb <= 0) return;
    mx_quant_rows_kernel<T><<<(unsigned)((nb + 255) / 256), 256, 0, st>>>(x, nb, q, s);
}

template void launch_mx_quant_rows<bf16>(const bf16*, int, int, uint8_t*, uint8_t*, hipStream_t);
template void launch_mx_quant_rows<float>(const float*, int, int, uint8_t*, uint8_t*, hipStream_t);

}  // namespace irodori
