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

// One wavefront per (b, s, h), lane = head dimension.  The head RMSNorm (norm.rs:60-74) and
// the interleaved half RoPE (rope.rs:82-135) as the QKV epilogue applies them.
template <typename T>
__global__ __launch_bounds__(256) void attn_op_stage_kernel(
    const float* __restrict__ q, const float* __restrict__ k, const float* __restrict__ v,
    const float* __restrict__ gate, const float* __restrict__ q_norm, const float* __restrict__ k_norm,
    const float* __restrict__ rope_cos, const float* __restrict__ rope_sin, int B, int S, int H, float eps,
    float q_scale, int vt_stride, T* __restrict__ Q, T* __restrict__ K, T* __restrict__ Vt, T* __restrict__ G) {
    const int d = threadIdx.x & 63;
    const int idx = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (idx >= B * S * H) return;
    const int h = idx % H, bs = idx / H, b = bs / S, s = bs % S;
    const size_t in = (size_t)idx * 64 + d;
    float yq = q[in], yk = k[in];
    if (q_norm) yq *= rsqrtf(wave_sum(yq * yq) * (1.f / 64.f) + eps) * q_norm[h * 64 + d];
    if (k_norm) yk *= rsqrtf(wave_sum(yk * yk) * (1.f / 64.f) + eps) * k_norm[h * 64 + d];
    if (h < H / 2) {
        const float c = rope_cos[(size_t)s * 32 + (d >> 1)], sn = rope_sin[(size_t)s * 32 + (d >> 1)];
        const float pq = __shfl_xor(yq, 1, 64), pk = __shfl_xor(yk, 1, 64);
        yq = (d & 1) ? pq * sn + yq * c : yq * c - pq * sn;
        yk = (d & 1) ? pk * sn + yk * c : yk * c - pk * sn;
    }
    const size_t o = (((size_t)b * H + h) * S + s) * 64 + d;
    Q[o] = from_f32<T>(yq * q_scale);
    K[o] = from_f32<T>(yk);
    Vt[(((size_t)b * H + h) * 64 + d) * vt_stride + vt_pos<T>(s)] = from_f32<T>(v[in]);
    const float gv = gate ? 1.f / (1.f + expf(-gate[in])) : 1.f;
    G[(size_t)bs * H * 64 + h * 64 + d] = from_f32<T>(gv);
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
    const int waves = B * S * H;
    attn_op_stage_kernel<T><<<(waves + 3) / 4, 256, 0, st>>>(q, k, v, gate, q_norm, k_norm, rope_cos, rope_sin, B, S,
                                                             H, eps, q_scale, vt_stride, Q, K, Vt, G);
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
