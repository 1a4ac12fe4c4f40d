// Speaker-KV scaling of the cached context (kv_scaling.rs:10-60): an HBM-bound elementwise
// pass over the device K / V^T copies the attention reads.  (The sampler's per-evaluation
// update runs in the output head, final_kernel.)
#include "common.hpp"
#include "kernels.hpp"

namespace irodori {

namespace {

// One thread per (row, head, key j, 8 dims) of K and the same for V^T.  V^T keys sit at
// vt_pos_bf16 (bf16_order) or vt_pos_f32.
template <typename T>
__global__ __launch_bounds__(256) void scale_ctx_aux_kernel(const T* __restrict__ src_k, const T* __restrict__ src_v,
                                                            T* __restrict__ dst_k, T* __restrict__ dst_v, int rows,
                                                            int rows_scaled, int H, int Dh, bool bf16_order, int T1,
                                                            int vs1, int t_ctx, int aux_start, float factor) {
    const int d8n = Dh / 8;
    const long total = (long)rows * H * T1 * d8n;
    const long idx = (long)blockIdx.x * 256 + threadIdx.x;
    if (idx >= total) return;
    const int d8 = (int)(idx % d8n);
    const long rhj = idx / d8n;
    const int j = (int)(rhj % T1);
    const long rh = rhj / T1;
    const int row = (int)(rh / H);
    const bool scale = row < rows_scaled && j >= aux_start && j < t_ctx;
    const bool copy = src_k != dst_k;
    if (!scale && !copy) return;
    const int pos = bf16_order ? vt_pos_bf16(j) : vt_pos_f32(j);
    for (int d = 8 * d8; d < 8 * d8 + 8; d++) {
        const size_t ko = ((size_t)rh * T1 + j) * Dh + d;
        const size_t vo = ((size_t)rh * Dh + d) * vs1 + pos;
        const float kf = static_cast<float>(src_k[ko]), vf = static_cast<float>(src_v[vo]);
        dst_k[ko] = scale ? static_cast<T>(kf * factor) : src_k[ko];
        dst_v[vo] = scale ? static_cast<T>(vf * factor) : src_v[vo];
    }
}

}  // namespace

template <typename T>
void launch_scale_ctx_aux(const T* src_k, const T* src_v, T* dst_k, T* dst_v, int rows, int rows_scaled, int H,
                          int Dh, bool bf16_order, int T1, int vs1, int t_ctx, int aux_start, float factor,
                          hipStream_t st) {
    const long total = (long)rows * H * T1 * (Dh / 8);
    scale_ctx_aux_kernel<T><<<(unsigned)((total + 255) / 256), 256, 0, st>>>(
        src_k, src_v, dst_k, dst_v, rows, rows_scaled, H, Dh, bf16_order, T1, vs1, t_ctx, aux_start, factor);
}

template void launch_scale_ctx_aux<bf16>(const bf16*, const bf16*, bf16*, bf16*, int, int, int, int, bool, int,
                                         int, int, int, float, hipStream_t);
template void launch_scale_ctx_aux<float>(const float*, const float*, float*, float*, int, int, int, int, bool, int,
                                          int, int, int, float, hipStream_t);

}  // namespace irodori
