// Element-wise and small kernels of the DACVAE decoder (codec/decoder.rs, layers.rs,
// bottleneck.rs).  The convolutions themselves run on the matrix-core GEMM
// (launch_gemm_conv); these kernels produce its operands:
//   * activations are channels-last [frames, Cp] (Cp = channels rounded up to 64, the
//     padded channels exactly zero), so a frame is one GEMM row;
//   * a convolution operand carries `halo` zero rows before and after the frames, which
//     are the convolution's zero padding: the implicit im2col of the GEMM never needs a
//     bounds test for the taps.
#include "common.hpp"
#include "kernels.hpp"

namespace irodori {

namespace {

template <typename T>
__device__ __forceinline__ float snake_c(float v, float a, float ar, float hc) {
    return snake_eval<T>(v, a, ar, hc);
}

template <typename T>
__device__ __forceinline__ void store8(T* p, const float (&v)[8]) {
    if constexpr (sizeof(T) == 2) {
        bf16x8 h;
#pragma unroll
        for (int i = 0; i < 8; i++) h[i] = static_cast<bf16>(v[i]);
        *reinterpret_cast<bf16x8*>(p) = h;
    } else {
        reinterpret_cast<float4*>(p)[0] = make_float4(v[0], v[1], v[2], v[3]);
        reinterpret_cast<float4*>(p)[1] = make_float4(v[4], v[5], v[6], v[7]);
    }
}

template <typename T>
__device__ __forceinline__ void load8(const T* p, float (&v)[8]) {
    if constexpr (sizeof(T) == 2) {
        const bf16x8 h = *reinterpret_cast<const bf16x8*>(p);
#pragma unroll
        for (int i = 0; i < 8; i++) v[i] = static_cast<float>(h[i]);
    } else {
        const float4 a = reinterpret_cast<const float4*>(p)[0], b = reinterpret_cast<const float4*>(p)[1];
        v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
        v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
    }
}

// quantizer.out_proj (bottleneck.rs:21-23, a k 1 Conv1d): s[r] = W lat[r - halo] + b over
// Cl latent channels, zeros in the halos.  W [Pp, Cl] and b [Pp] f32, zero past the real
// channels.  A workgroup owns kCodecInRows operand rows and 256 output channels: the rows'
// latents sit in LDS (read as broadcasts), and thread o walks weight row o once, feeding
// every row's accumulator in the order c = 0 .. Cl - 1 before adding b[o].
constexpr int kCodecInRows = 8;

template <typename T>
__global__ __launch_bounds__(256) void codec_in_kernel(const float* __restrict__ lat, int frames, int Cl,
                                                       const float* __restrict__ w, const float* __restrict__ b,
                                                       int Pp, int halo, T* __restrict__ s) {
    extern __shared__ float ls[];  // [kCodecInRows][Cl]
    const int r0 = blockIdx.x * kCodecInRows, rows = frames + 2 * halo;
    const int o = blockIdx.y * 256 + threadIdx.x;
    for (int i = threadIdx.x; i < kCodecInRows * Cl; i += 256) {
        const int t = r0 + i / Cl - halo;
        ls[i] = (t >= 0 && t < frames) ? lat[(size_t)t * Cl + i % Cl] : 0.f;
    }
    __syncthreads();
    if (o >= Pp) return;
    float acc[kCodecInRows];
#pragma unroll
    for (int r = 0; r < kCodecInRows; r++) acc[r] = 0.f;
    const float* wr = w + (size_t)o * Cl;
    for (int c = 0; c < Cl; c++) {
        const float wc = wr[c];
#pragma unroll
        for (int r = 0; r < kCodecInRows; r++) acc[r] = fmaf(wc, ls[r * Cl + c], acc[r]);
    }
    const float bo = b[o];
#pragma unroll
    for (int r = 0; r < kCodecInRows; r++) {
        const int t = r0 + r - halo;
        if (r0 + r < rows) s[(size_t)(r0 + r) * Pp + o] = static_cast<T>(t >= 0 && t < frames ? acc[r] + bo : 0.f);
    }
}

// WmHead (decoder.rs WmHead::forward) fused with its Snake: wav[t] = tanh(b + sum_j sum_c
// w[j, c] Snake(x[t + j - 3, c])) over x [L, Cp] f32 (zero padding outside [0, L)), taps
// w [7, Cp] f32 (w[j Cp + c] = weight[0, c, j], zero past the real channels).  A workgroup
// owns 256 frames: its waves reduce the 262 rows those frames read to per-tap dot products
// p[row][j] in LDS (4 lanes per row, each lane Cp / 4 channels in float4 loads), then
// thread t sums its seven taps.  The taps and Snake constants sit in LDS.  Cp <= 256.
template <typename T>
__global__ __launch_bounds__(256) void codec_head_kernel(const float* __restrict__ x, int L, int Cp,
                                                         const float* __restrict__ alpha, const float* __restrict__ w,
                                                         const float* __restrict__ b, float* __restrict__ wav) {
    constexpr int FR = 256, ROWS = FR + 6;
    __shared__ float p[ROWS][8];
    __shared__ float4 wl[7][64], al[3][64];
    const int t0 = blockIdx.x * FR, tid = threadIdx.x, q = tid & 3, grp = tid >> 2;  // 64 row groups
    const int c4n = Cp / 4;  // float4 columns
    for (int i = tid; i < 7 * c4n; i += 256) wl[i / c4n][i % c4n] = reinterpret_cast<const float4*>(w)[i];
    for (int i = tid; i < 3 * c4n; i += 256) al[i / c4n][i % c4n] = reinterpret_cast<const float4*>(alpha)[i];
    __syncthreads();
    const int per = c4n / 4;  // float4 columns per lane: q, q + 4, ...
    for (int rr = grp; rr < ROWS; rr += 64) {
        const int f = t0 - 3 + rr;
        float acc[7] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
        if (f >= 0 && f < L) {
            const float4* xr = reinterpret_cast<const float4*>(x + (size_t)f * Cp);
            for (int k = 0; k < per; k++) {
                const int c4 = q + 4 * k;
                const float4 xv = xr[c4], av = al[0][c4], ar = al[1][c4], hc = al[2][c4];
                const float s0 = snake_c<T>(xv.x, av.x, ar.x, hc.x), s1 = snake_c<T>(xv.y, av.y, ar.y, hc.y);
                const float s2 = snake_c<T>(xv.z, av.z, ar.z, hc.z), s3 = snake_c<T>(xv.w, av.w, ar.w, hc.w);
#pragma unroll
                for (int j = 0; j < 7; j++) {
                    const float4 wv = wl[j][c4];
                    acc[j] = fmaf(wv.x, s0, fmaf(wv.y, s1, fmaf(wv.z, s2, fmaf(wv.w, s3, acc[j]))));
                }
            }
        }
#pragma unroll
        for (int j = 0; j < 7; j++) {
            acc[j] += __shfl_xor(acc[j], 1, 4);
            acc[j] += __shfl_xor(acc[j], 2, 4);
        }
        if (q == 0) {
#pragma unroll
            for (int j = 0; j < 7; j++) p[rr][j] = acc[j];
        }
    }
    __syncthreads();
    const int t = t0 + tid;
    if (t >= L) return;
    float y = b ? b[0] : 0.f;
#pragma unroll
    for (int j = 0; j < 7; j++) y += p[tid + j][j];
    wav[t] = tanhf(y);
}

// Zero the halo rows [0, halo) and [halo + L, L + 2 halo) of an operand [L + 2 halo, Cp].
template <typename T>
__global__ __launch_bounds__(256) void zero_halo_kernel(T* __restrict__ s, int L, int Cp, int halo) {
    const int c8 = Cp / 8;
    const int idx = blockIdx.x * 256 + threadIdx.x;
    if (idx >= 2 * halo * c8) return;
    int r = idx / c8;
    if (r >= halo) r += L;
    float z[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    store8<T>(s + (size_t)r * Cp + (idx % c8) * 8, z);
}

template <typename T>
__global__ __launch_bounds__(256) void cvt_f32_kernel(const float* __restrict__ src, long n, T* __restrict__ dst) {
    const long i = (long)blockIdx.x * 256 + threadIdx.x;
    if (i < n) dst[i] = from_f32<T>(src[i]);
}

inline unsigned blocks_for(long n) { return (unsigned)((n + 255) / 256); }

}  // namespace

template <typename T>
void launch_codec_in(const float* lat, int frames, int Cl, const float* w, const float* b, int Pp, int halo, T* s,
                     hipStream_t st) {
    const int rows = frames + 2 * halo;
    if (rows <= 0 || Pp <= 0) return;
    const dim3 grid((unsigned)((rows + kCodecInRows - 1) / kCodecInRows), (unsigned)((Pp + 255) / 256));
    codec_in_kernel<T><<<grid, 256, sizeof(float) * kCodecInRows * Cl, st>>>(lat, frames, Cl, w, b, Pp, halo, s);
}

template <typename T>
void launch_codec_head(const float* x, int L, int Cp, const float* alpha, const float* w, const float* b, float* wav,
                       hipStream_t st) {
    if (L > 0) codec_head_kernel<T><<<blocks_for(L), 256, 0, st>>>(x, L, Cp, alpha, w, b, wav);
}

template <typename T>
void launch_codec_zero_halo(T* s, int L, int Cp, int halo, hipStream_t st) {
    const long n = 2L * halo * (Cp / 8);
    if (n > 0) zero_halo_kernel<T><<<blocks_for(n), 256, 0, st>>>(s, L, Cp, halo);
}

template <typename T>
void launch_cvt_f32(const float* src, long n, T* dst, hipStream_t st) {
    if (n > 0) cvt_f32_kernel<T><<<blocks_for(n), 256, 0, st>>>(src, n, dst);
}

#define IRO_CODEC_INST(T)                                                                                   \
    template void launch_codec_in<T>(const float*, int, int, const float*, const float*, int, int, T*,       \
                                     hipStream_t);                                                          \
    template void launch_codec_head<T>(const float*, int, int, const float*, const float*, const float*, float*, \
                                       hipStream_t);                                                          \
    template void launch_cvt_f32<T>(const float*, long, T*, hipStream_t);                                    \
    template void launch_codec_zero_halo<T>(T*, int, int, int, hipStream_t);
IRO_CODEC_INST(bf16)
IRO_CODEC_INST(float)
#undef IRO_CODEC_INST

}  // namespace irodori
