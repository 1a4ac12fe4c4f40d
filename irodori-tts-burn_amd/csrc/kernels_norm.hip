// HBM-bound row kernels: RMSNorm, adaLN modulation, in_proj + modulation, output head
// with the Joint-CFG combine and Euler update.  One wavefront per row, 4 rows per
// 256-thread workgroup; rows are read with 16-byte loads and reduced in registers with
// cross-lane shuffles (no LDS), so each row is read from HBM exactly once.
#include "common.hpp"
#include "kernels.hpp"

namespace irodori {

namespace {

constexpr int kRowsPerBlock = 4;

__device__ __forceinline__ int mod_vec(const ModTable& mt, int b) {
    int step = mt.step ? *mt.step : 0;
    return step * mt.step_stride + b / mt.rows_per_vec;
}

// Pointer to (shift, scale, gate) of (layer, kind) for batch row b.
__device__ __forceinline__ const float* mod_base(const ModTable& mt, int b, int layer, int kind,
                                                int D) {
    return mt.tab + ((size_t)mod_vec(mt, b) * mt.layers * 6 + (size_t)layer * 6 + kind * 3) * D;
}

template <typename T>
__device__ __forceinline__ void store4(T* p, float a, float b, float c, float d);
template <>
__device__ __forceinline__ void store4<float>(float* p, float a, float b, float c, float d) {
    *reinterpret_cast<float4*>(p) = make_float4(a, b, c, d);
}
template <>
__device__ __forceinline__ void store4<bf16>(bf16* p, float a, float b, float c, float d) {
    typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
    bf16x4 v = {static_cast<bf16>(a), static_cast<bf16>(b), static_cast<bf16>(c),
                static_cast<bf16>(d)};
    *reinterpret_cast<bf16x4*>(p) = v;
}

// Row RMSNorm with weight (rms_norm.rs:161-175 semantics), generic D.
__global__ __launch_bounds__(256) void rms_norm_op_kernel(const float* __restrict__ x,
                                                          const float* __restrict__ w, int rows,
                                                          int D, float eps,
                                                          float* __restrict__ y) {
    int row = blockIdx.x * kRowsPerBlock + threadIdx.x / 64, lane = threadIdx.x % 64;
    if (row >= rows) return;
    const float* xr = x + (size_t)row * D;
    float ss = 0.f;
    for (int d = lane; d < D; d += 64) ss += xr[d] * xr[d];
    ss = wave_sum(ss);
    float rms = sqrtf(ss / (float)D + eps);
    for (int d = lane; d < D; d += 64) y[(size_t)row * D + d] = xr[d] / rms * w[d];
}

// fused_adaln semantics (fused_adaln.rs:223-251), generic D.
__global__ __launch_bounds__(256) void fused_adaln_op_kernel(
    const float* __restrict__ x, const float* __restrict__ scale,
    const float* __restrict__ shift, int B, int S, int D, float eps, float* __restrict__ y) {
    int row = blockIdx.x * kRowsPerBlock + threadIdx.x / 64, lane = threadIdx.x % 64;
    if (row >= B * S) return;
    int b = row / S;
    const float* xr = x + (size_t)row * D;
    float ss = 0.f;
    for (int d = lane; d < D; d += 64) ss += xr[d] * xr[d];
    ss = wave_sum(ss);
    float rms = sqrtf(ss / (float)D + eps);
    for (int d = lane; d < D; d += 64)
        y[(size_t)row * D + d] = xr[d] / rms * (1.f + scale[b * D + d]) + shift[b * D + d];
}

// Model adaLN modulation: h = x / rms * (1 + scale) + shift (norm.rs:160-169).
// D % 4 == 0; each lane owns float4 chunks lane*4 + 256*j.
template <typename T, int NCH>
__global__ __launch_bounds__(256) void norm_mod_kernel(const float* __restrict__ x,
                                                       T* __restrict__ h, int M, int S, int D,
                                                       float eps, ModTable mt, int layer,
                                                       int kind) {
    int row = blockIdx.x * kRowsPerBlock + threadIdx.x / 64, lane = threadIdx.x % 64;
    if (row >= M) return;
    const float* xr = x + (size_t)row * D;
    float4 v[NCH];
    float ss = 0.f;
#pragma unroll
    for (int j = 0; j < NCH; j++) {
        int d = lane * 4 + 256 * j;
        v[j] = d < D ? *reinterpret_cast<const float4*>(xr + d) : make_float4(0, 0, 0, 0);
        ss += v[j].x * v[j].x + v[j].y * v[j].y + v[j].z * v[j].z + v[j].w * v[j].w;
    }
    ss = wave_sum(ss);
    float rms = sqrtf(ss / (float)D + eps);
    const float* base = mod_base(mt, row / S, layer, kind, D);
    const float* shift = base;
    const float* scale = base + D;
#pragma unroll
    for (int j = 0; j < NCH; j++) {
        int d = lane * 4 + 256 * j;
        if (d >= D) break;
        float4 sc = *reinterpret_cast<const float4*>(scale + d);
        float4 sh = *reinterpret_cast<const float4*>(shift + d);
        store4<T>(h + (size_t)row * D + d, v[j].x / rms * (1.f + sc.x) + sh.x,
                  v[j].y / rms * (1.f + sc.y) + sh.y, v[j].z / rms * (1.f + sc.z) + sh.z,
                  v[j].w / rms * (1.f + sc.w) + sh.w);
    }
}

// in_proj (x = x_src @ W_in + b_in, dit/model.rs:370) fused with the first adaLN.
template <typename T, int NCH>
__global__ __launch_bounds__(256) void inproj_norm_kernel(
    const float* __restrict__ x_src, int rows_per_src, const float* __restrict__ in_w,
    const float* __restrict__ in_b, float* __restrict__ x, T* __restrict__ h, int M, int S, int P,
    int D, float eps, ModTable mt) {
    int row = blockIdx.x * kRowsPerBlock + threadIdx.x / 64, lane = threadIdx.x % 64;
    if (row >= M) return;
    int b = row / S, s = row % S;
    const float* src = x_src + ((size_t)(b / rows_per_src) * S + s) * P;
    float4 v[NCH];
    float ss = 0.f;
#pragma unroll
    for (int j = 0; j < NCH; j++) {
        int d = lane * 4 + 256 * j;
        float4 acc = make_float4(0, 0, 0, 0);
        if (d < D) {
            acc = *reinterpret_cast<const float4*>(in_b + d);
            for (int p = 0; p < P; p++) {
                float a = src[p];
                float4 wv = *reinterpret_cast<const float4*>(in_w + (size_t)p * D + d);
                acc.x += a * wv.x; acc.y += a * wv.y; acc.z += a * wv.z; acc.w += a * wv.w;
            }
            *reinterpret_cast<float4*>(x + (size_t)row * D + d) = acc;
        }
        v[j] = acc;
        ss += acc.x * acc.x + acc.y * acc.y + acc.z * acc.z + acc.w * acc.w;
    }
    ss = wave_sum(ss);
    float rms = sqrtf(ss / (float)D + eps);
    const float* base = mod_base(mt, b, 0, 0, D);
    const float* shift = base;
    const float* scale = base + D;
#pragma unroll
    for (int j = 0; j < NCH; j++) {
        int d = lane * 4 + 256 * j;
        if (d >= D) break;
        float4 sc = *reinterpret_cast<const float4*>(scale + d);
        float4 sh = *reinterpret_cast<const float4*>(shift + d);
        store4<T>(h + (size_t)row * D + d, v[j].x / rms * (1.f + sc.x) + sh.x,
                  v[j].y / rms * (1.f + sc.y) + sh.y, v[j].z / rms * (1.f + sc.z) + sh.z,
                  v[j].w / rms * (1.f + sc.w) + sh.w);
    }
}

// Output head: one wavefront per latent frame s handles every batch row of that frame, two
// rows at a time, so the Joint-CFG combine of rows (2u, 2u+1) and the Euler update happen
// in registers.  v[b,s,p] = (sum_d x[b,s,d] * W'[p,d]) / rms(x[b,s,:]) + b_out[p] with
// W' = out_norm.weight (.) W_out^T folded at ingest — the same product as
// out_proj(out_norm(x)) (norm.rs:25-39, dit/model.rs:391-392).  Each lane accumulates its
// D/64 columns for all PT outputs in registers; the cross-lane sums go through a padded
// [row][p][65] LDS tile (conflict-free writes and reads).
template <int PT>
__global__ __launch_bounds__(64) void final_kernel(FinalArgs a) {
    __shared__ float red[2][PT][65];
    const int s = blockIdx.x, lane = threadIdx.x;
    const int D = a.D, P = a.P;
    const int step = a.step ? *a.step : 0;
    float dt = 0.f;
    int cfg_on = 0;
    if (a.mode == 1) {
        dt = a.t_sched[step + 1] - a.t_sched[step];
        cfg_on = a.cfg_on[step];
    }
    for (int b0 = 0; b0 < a.B; b0 += 2) {
        const bool two = b0 + 1 < a.B;
        const float* x0 = a.x + ((size_t)b0 * a.S + s) * D;
        const float* x1 = a.x + ((size_t)(two ? b0 + 1 : b0) * a.S + s) * D;
        float part0[PT], part1[PT];
#pragma unroll
        for (int p = 0; p < PT; p++) { part0[p] = 0.f; part1[p] = 0.f; }
        float ss0 = 0.f, ss1 = 0.f;
        for (int d = lane; d < D; d += 64) {
            float u0 = x0[d], u1 = x1[d];
            ss0 += u0 * u0;
            ss1 += u1 * u1;
#pragma unroll
            for (int p = 0; p < PT; p++) {
                float w = p < P ? a.out_wT[(size_t)p * D + d] : 0.f;
                part0[p] += u0 * w;
                part1[p] += u1 * w;
            }
        }
        ss0 = wave_sum(ss0);
        ss1 = wave_sum(ss1);
#pragma unroll
        for (int p = 0; p < PT; p++) {
            red[0][p][lane] = part0[p];
            red[1][p][lane] = part1[p];
        }
        __syncthreads();
        float v0 = 0.f, v1 = 0.f;
        if (lane < P) {
            for (int l = 0; l < 64; l++) {
                v0 += red[0][lane][l];
                v1 += red[1][lane][l];
            }
            v0 = v0 / sqrtf(ss0 / (float)D + a.eps) + a.out_b[lane];
            v1 = v1 / sqrtf(ss1 / (float)D + a.eps) + a.out_b[lane];
        }
        __syncthreads();
        if (lane >= P) continue;
        if (a.mode == 0) {
            a.v_out[((size_t)b0 * a.S + s) * P + lane] = v0;
            if (two) a.v_out[((size_t)(b0 + 1) * a.S + s) * P + lane] = v1;
        } else {
            // euler_sampler.rs:467 (v_c + (v_c - v_u) * scale) and :714 (x += v * dt)
            float vv = cfg_on ? v0 + (v0 - v1) * a.scale : v0;
            float* xt = a.xt + ((size_t)(b0 / 2) * a.S + s) * P + lane;
            *xt = *xt + vv * dt;
        }
    }
}

__global__ void step_advance_kernel(int* step) {
    if (threadIdx.x == 0) *step = *step + 1;
}

__global__ void scale_copy_kernel(const float* __restrict__ src, float* __restrict__ dst, int n,
                                  float s) {
    int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) dst[i] = src[i] * s;
}

}  // namespace

void launch_rms_norm_op(const float* x, const float* w, int rows, int D, float eps, float* y,
                        hipStream_t st) {
    int grid = (rows + kRowsPerBlock - 1) / kRowsPerBlock;
    rms_norm_op_kernel<<<grid, 256, 0, st>>>(x, w, rows, D, eps, y);
}

void launch_fused_adaln_op(const float* x, const float* scale, const float* shift, int B, int S,
                           int D, float eps, float* y, hipStream_t st) {
    int grid = (B * S + kRowsPerBlock - 1) / kRowsPerBlock;
    fused_adaln_op_kernel<<<grid, 256, 0, st>>>(x, scale, shift, B, S, D, eps, y);
}

template <typename T>
void launch_norm_mod(const float* x, T* h, int M, int S, int D, float eps, ModTable mt,
                     int layer, int kind, hipStream_t st) {
    int grid = (M + kRowsPerBlock - 1) / kRowsPerBlock;
    int nch = (D + 255) / 256;
    if (nch <= 1)
        norm_mod_kernel<T, 1><<<grid, 256, 0, st>>>(x, h, M, S, D, eps, mt, layer, kind);
    else if (nch <= 2)
        norm_mod_kernel<T, 2><<<grid, 256, 0, st>>>(x, h, M, S, D, eps, mt, layer, kind);
    else if (nch <= 4)
        norm_mod_kernel<T, 4><<<grid, 256, 0, st>>>(x, h, M, S, D, eps, mt, layer, kind);
    else
        norm_mod_kernel<T, 8><<<grid, 256, 0, st>>>(x, h, M, S, D, eps, mt, layer, kind);
}

template <typename T>
void launch_inproj_norm(const float* x_src, int rows_per_src, const float* in_w,
                        const float* in_b, float* x, T* h, int M, int S, int P, int D, float eps,
                        ModTable mt, hipStream_t st) {
    int grid = (M + kRowsPerBlock - 1) / kRowsPerBlock;
    int nch = (D + 255) / 256;
#define IRO_INPROJ(N)                                                                      \
    inproj_norm_kernel<T, N><<<grid, 256, 0, st>>>(x_src, rows_per_src, in_w, in_b, x, h, M, \
                                                   S, P, D, eps, mt)
    if (nch <= 1) IRO_INPROJ(1);
    else if (nch <= 2) IRO_INPROJ(2);
    else if (nch <= 4) IRO_INPROJ(4);
    else IRO_INPROJ(8);
#undef IRO_INPROJ
}

template void launch_norm_mod<float>(const float*, float*, int, int, int, float, ModTable, int,
                                     int, hipStream_t);
template void launch_norm_mod<bf16>(const float*, bf16*, int, int, int, float, ModTable, int,
                                    int, hipStream_t);
template void launch_inproj_norm<float>(const float*, int, const float*, const float*, float*,
                                        float*, int, int, int, int, float, ModTable,
                                        hipStream_t);
template void launch_inproj_norm<bf16>(const float*, int, const float*, const float*, float*,
                                       bf16*, int, int, int, int, float, ModTable, hipStream_t);

void launch_final(const FinalArgs& a, hipStream_t st) {
    if (a.P <= 8) final_kernel<8><<<a.S, 64, 0, st>>>(a);
    else if (a.P <= 16) final_kernel<16><<<a.S, 64, 0, st>>>(a);
    else if (a.P <= 32) final_kernel<32><<<a.S, 64, 0, st>>>(a);
    else final_kernel<64><<<a.S, 64, 0, st>>>(a);
}

void launch_step_advance(int* step, hipStream_t st) { step_advance_kernel<<<1, 64, 0, st>>>(step); }

void launch_scale_copy(const float* src, float* dst, int n, float s, hipStream_t st) {
    scale_copy_kernel<<<(n + 255) / 256, 256, 0, st>>>(src, dst, n, s);
}

}  // namespace irodori
