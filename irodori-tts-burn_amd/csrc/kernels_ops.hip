// Small kernels of the isolated block operators (irodori_op_joint_attention /
// irodori_op_swiglu_mlp): staging the caller's attention operands into the layouts the
// model's QKV+gate epilogue writes, widening the gated attention output to f32, and placing
// caller modulation vectors in the context's table.
#include "common.hpp"
#include "kernels.hpp"

namespace irodori {

namespace {

template <typename T>
__device__ __forceinline__ int vt_pos(int s) {
    return sizeof(T) == 2 ? vt_pos_bf16(s) : vt_pos_f32(s);
}

// Column of the 64-key block that V^T position p holds (the inverse of vt_pos; both key
// orders only permute keys inside aligned groups of 16 (bf16) or 32 (f32)).
template <typename T>
__device__ __forceinline__ int vt_src(int p) {
    if (sizeof(T) == 2) return vt_pos_bf16(p);  // a swap of key bits 2 and 3: its own inverse
    const int pp = p & 31;
    return (p & ~31) | (((pp >> 2) & 1) * 16 + (pp >> 3) * 4 + (pp & 3));
}

// One block per (b, h, 64 tokens): 8 wavefronts x 8 tokens, lane = head dimension, the
// inputs of a wavefront's 8 tokens loaded together.  The head RMSNorm (norm.rs:60-74) and the interleaved
// half RoPE (rope.rs:82-135) as the QKV epilogue applies them.  V goes through LDS so that
// each V^T row (b, h, d) leaves as one contiguous run per 16 keys; keys past S (up to the
// 64-key boundary) are written as zeros.
template <typename T>
__global__ __launch_bounds__(512) void attn_op_stage_kernel(
    const float* __restrict__ q, const float* __restrict__ k, const float* __restrict__ v,
    const float* __restrict__ gate, const float* __restrict__ q_norm, const float* __restrict__ k_norm,
    const float* __restrict__ rope_cos, const float* __restrict__ rope_sin, int B, int S, int H, float eps,
    float q_scale, int vt_stride, T* __restrict__ Q, T* __restrict__ K, T* __restrict__ Vt, T* __restrict__ G) {
    __shared__ float vs[64][65];
    const int d = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int s0 = blockIdx.x * 64, h = blockIdx.y, b = blockIdx.z;
    const float qn = q_norm ? q_norm[h * 64 + d] : 1.f, kn = k_norm ? k_norm[h * 64 + d] : 1.f;
    {
        constexpr int i0 = 0;
        float xq[8], xk[8], xv[8], xg[8], rc[8], rs[8];
        const bool rope = h < H / 2;
#pragma unroll
        for (int u = 0; u < 8; u++) {
            const int s = s0 + wave * 8 + u, sc = s < S ? s : S - 1;
            const size_t in = (((size_t)b * S + sc) * H + h) * 64 + d;
            xq[u] = q[in];
            xk[u] = k[in];
            xv[u] = v[in];
            xg[u] = gate ? gate[in] : 0.f;
            rc[u] = rope ? rope_cos[(size_t)sc * 32 + (d >> 1)] : 1.f;
            rs[u] = rope ? rope_sin[(size_t)sc * 32 + (d >> 1)] : 0.f;
        }
#pragma unroll
        for (int u = 0; u < 8; u++) {
            const int sl = wave * 8 + i0 + u, s = s0 + sl;
            if (s >= S) {  // wave-uniform
                vs[sl][d] = 0.f;
                continue;
            }
            float yq = xq[u], yk = xk[u];
            if (q_norm) yq *= rsqrtf(wave_sum(yq * yq) * (1.f / 64.f) + eps) * qn;
            if (k_norm) yk *= rsqrtf(wave_sum(yk * yk) * (1.f / 64.f) + eps) * kn;
            if (rope) {
                const float c = rc[u], sn = rs[u];
                const float pq = __shfl_xor(yq, 1, 64), pk = __shfl_xor(yk, 1, 64);
                yq = (d & 1) ? pq * sn + yq * c : yq * c - pq * sn;
                yk = (d & 1) ? pk * sn + yk * c : yk * c - pk * sn;
            }
            const size_t o = (((size_t)b * H + h) * S + s) * 64 + d;
            Q[o] = from_f32<T>(yq * q_scale);
            K[o] = from_f32<T>(yk);
            const float gv = gate ? 1.f / (1.f + expf(-xg[u])) : 1.f;
            G[((size_t)b * S + s) * H * 64 + h * 64 + d] = from_f32<T>(gv);
            vs[sl][d] = xv[u];
        }
    }
    __syncthreads();
    // V^T row (b, h, dd), positions 8 seg .. 8 seg + 7 of this 64-key block.
    const int dd = threadIdx.x >> 3, seg = threadIdx.x & 7;
    T row[8];
#pragma unroll
    for (int j = 0; j < 8; j++) row[j] = from_f32<T>(vs[vt_src<T>(8 * seg + j)][dd]);
    T* dst = Vt + (((size_t)b * H + h) * 64 + dd) * vt_stride + s0 + 8 * seg;
    constexpr int PER = 16 / sizeof(T);  // elements per 16-byte store
#pragma unroll
    for (int j = 0; j < 8; j += PER) *reinterpret_cast<uint4*>(dst + j) = *reinterpret_cast<const uint4*>(row + j);
}

template <typename T>
__global__ __launch_bounds__(256) void to_f32_kernel(const T* __restrict__ src, long n, float* __restrict__ dst) {
    for (long i = blockIdx.x * 256L + threadIdx.x; i < n; i += (long)gridDim.x * 256) dst[i] = to_f32(src[i]);
}

__global__ __launch_bounds__(256) void put_mod_vectors_kernel(const float* __restrict__ shift,
                                                              const float* __restrict__ scale,
                                                              const float* __restrict__ gate, int D, int layers,
                                                              int layer, int kind, float* __restrict__ tab) {
    const int b = blockIdx.y;
    float* row = tab + ((size_t)b * layers * 6 + (size_t)layer * 6 + kind * 3) * D;
    for (int d = blockIdx.x * 256 + threadIdx.x; d < D; d += gridDim.x * 256) {
        row[d] = shift[(size_t)b * D + d];
        row[D + d] = scale[(size_t)b * D + d];
        row[2 * D + d] = gate[(size_t)b * D + d];
    }
}

}  // namespace

template <typename T>
void launch_attn_op_stage(const float* q, const float* k, const float* v, const float* gate, const float* q_norm,
                          const float* k_norm, const float* rope_cos, const float* rope_sin, int B, int S, int H,
                          float eps, float q_scale, int vt_stride, T* Q, T* K, T* Vt, T* G, hipStream_t st) {
    // vt_stride is S rounded up to 64: every block's V^T columns lie inside it.
    const dim3 grid((S + 63) / 64, H, B);
    attn_op_stage_kernel<T><<<grid, 512, 0, st>>>(q, k, v, gate, q_norm, k_norm, rope_cos, rope_sin, B, S, H, eps,
                                                  q_scale, vt_stride, Q, K, Vt, G);
}
template void launch_attn_op_stage<bf16>(const float*, const float*, const float*, const float*, const float*,
                                         const float*, const float*, const float*, int, int, int, float, float, int,
                                         bf16*, bf16*, bf16*, bf16*, hipStream_t);
template void launch_attn_op_stage<float>(const float*, const float*, const float*, const float*, const float*,
                                          const float*, const float*, const float*, int, int, int, float, float, int,
                                          float*, float*, float*, float*, hipStream_t);

template <typename T>
void launch_to_f32(const T* src, long n, float* dst, hipStream_t st) {
    long blocks = (n + 255) / 256;
    to_f32_kernel<T><<<(unsigned)(blocks < 4096 ? blocks : 4096), 256, 0, st>>>(src, n, dst);
}
template void launch_to_f32<bf16>(const bf16*, long, float*, hipStream_t);
template void launch_to_f32<float>(const float*, long, float*, hipStream_t);

void launch_put_mod_vectors(const float* shift, const float* scale, const float* gate, int B, int D, int layers,
                            int layer, int kind, float* tab, hipStream_t st) {
    put_mod_vectors_kernel<<<dim3((D + 255) / 256, B), 256, 0, st>>>(shift, scale, gate, D, layers, layer, kind, tab);
}

}  // namespace irodori
