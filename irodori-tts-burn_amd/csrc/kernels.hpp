// Host-side launchers for the gfx950 kernels (one .hip file per kernel family).
// All launchers validate nothing themselves: callers (context.hip, the op entry points)
// check shapes against what each kernel's grid assumes before launching.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace irodori {

// Where the adaLN modulation vectors of a forward live: a table of rows
// [vec][layer][kind(attn,mlp)][chunk(shift,scale,gate)][D] (gate already tanh'd).
// Row index for batch row b: vec = (*step) * step_stride + (b / rows_per_vec).
struct ModTable {
    const float* tab;
    const int* step;   // device step counter (0 for single forwards)
    int step_stride;   // vectors per step
    int rows_per_vec;  // batch rows sharing one vector
    int layers;
};

// Position of latent/context key s inside a V^T row.  bf16 path (32x32x16 attention):
// bits 2 and 3 of the key index swapped; f32 path (16x16 attention): keys permuted inside
// each 32-key group.  Both are involutions on aligned groups, so padding stays in place.
__host__ __device__ inline int vt_pos_bf16(int s) { return (s & ~12) | ((s & 4) << 1) | ((s & 8) >> 1); }
__host__ __device__ inline int vt_pos_f32(int s) {
    int kk = s & 31;
    return (s & ~31) | (((kk & 15) >> 2) * 8 + (kk >> 4) * 4 + (kk & 3));
}

// ---- kernels_norm.hip ------------------------------------------------------------------
void launch_rms_norm_op(const float* x, const float* w, int rows, int D, float eps, float* y,
                        hipStream_t st);
void launch_fused_adaln_op(const float* x, const float* scale, const float* shift, int B, int S,
                           int D, float eps, float* y, hipStream_t st);
// h = x / sqrt(mean(x^2)+eps) * (1 + scale) + shift for (layer, kind) of the table.
template <typename T>
void launch_norm_mod(const float* x, T* h, int M, int S, int D, float eps, ModTable mt,
                     int layer, int kind, hipStream_t st);
// x = x_src[row] @ in_w + in_b (in_proj), then h = norm_mod(x) for (layer 0, attn).
template <typename T>
void launch_inproj_norm(const float* x_src, int rows_per_src, const float* in_w,
                        const float* in_b, float* x, T* h, int M, int S, int P, int D,
                        float eps, ModTable mt, hipStream_t st);

// Output head.  mode 0: v[b,s,:] = out_proj(out_norm(x[b,s,:])).
// mode 1 (Joint CFG + Euler): per utterance u, v = v_c + scale (v_c - v_u) when the step
// is guided (else v_c), then x_t[u,s,:] += v * (t[step+1] - t[step]).
struct FinalArgs {
    const float* x;
    const float* norm_w;
    const float* out_wT;  // [P, D] = (out_norm.weight (.) W_out)^T
    const float* out_b;   // [P]
    int B, S, D, P;
    float eps;
    int mode;
    float* v_out;        // mode 0: [B,S,P]
    float* xt;           // mode 1: [U,S,P]
    const float* t_sched;  // [steps+1]
    const int* cfg_on;     // [steps]
    const int* step;
    float scale;
};
void launch_final(const FinalArgs& a, hipStream_t st);
void launch_step_advance(int* step, hipStream_t st);
void launch_scale_copy(const float* src, float* dst, int n, float s, hipStream_t st);

// ---- kernels_cond.hip ------------------------------------------------------------------
struct VecLinJob {
    const float* X;  // [nvec, ldx]
    const float* W;  // [K, N] row-major
    const float* bias;  // [N] or null
    const float* R;  // residual [nvec, ldr] or null
    float* Y;        // [nvec, ldy]
    int ldx, ldr, ldy, K, N;
    int act_in;   // 0 none, 1 silu
    int act_out;  // 0 none, 1 silu, 2 tanh
};
void launch_timestep_embedding(const float* t, int nvec, int t_dim, float* out, hipStream_t st);
void launch_vec_linear(const VecLinJob* d_jobs, int njobs, int nvec, int max_n, hipStream_t st);

// ---- kernels_gemm.hip ------------------------------------------------------------------
enum GemmEpi { EPI_STORE = 0, EPI_RESID = 1, EPI_SWIGLU = 2, EPI_QKVG = 3 };
template <typename T>
struct GemmArgs {
    const T* A;   // [M, K] row-major
    const T* W;   // [N, K] row-major (K contiguous)
    int M, N, K;
    // EPI_STORE: C [M, N] f32
    float* C;
    // EPI_RESID: x[m, n] += gate[vec(b), n] * acc, b = m / S
    float* x;
    ModTable mt;
    int layer, kind;
    int S;
    // EPI_SWIGLU: U [M, N/2] = silu(acc_1) * acc_3 (W rows interleaved in 32-row groups)
    T* U;
    // EPI_QKVG: N = 4 * D; q/k head-normed (+ half RoPE), v raw, gate sigmoid.
    T* Q;  // [B, H, S, Dh]
    T* Kd; // [B, H, S, Dh]
    T* Vd; // V^T [B, H, Dh, vt_stride], key s at vt_pos_bf16 / vt_pos_f32 by dtype
    int vt_stride;  // multiple of 64, >= S
    float q_scale;  // q multiplier (Dh^-1/2 * log2 e) applied after norm + RoPE
    T* G;  // [M, D]
    const float* q_norm;  // [H, Dh]
    const float* k_norm;
    const float* rope_cos;  // [S, Dh/2]
    const float* rope_sin;
    int H, D;
    float eps;
};
template <typename T>
int launch_gemm(int epi, const GemmArgs<T>& a, hipStream_t st);

// ---- kernels_attn.hip ------------------------------------------------------------------
template <typename T>
struct AttnArgs {
    const T* Q;        // [B, H, Sq, Dh]
    // segment 0 (latent self keys): [B, H, seg0_stride, Dh], len0 keys, no mask
    const T* K0;
    const T* V0;
    int len0, stride0;
    const float* mask0;  // optional [B, len0]; value < 0.5 = masked out
    // optional [B, ceil(len0/64)]: bit k of tile t set iff latent key 64 t + k attends
    // (launch_attention32; required there together with mask0)
    const unsigned long long* bits0;
    // segment 1 (cached context keys): [B, H, stride1, Dh], len1 keys
    const T* K1;
    const T* V1;
    int len1, stride1;
    const float* mask1;   // optional [B, stride1]; value < 0.5 = masked out
    const int* tile_on1;  // [B, ceil(stride1/64)] nonzero if the 64-key tile has a valid key
    // [B, ceil(stride1/64)]: bit k of tile t set iff key 64 t + k is valid (launch_attention32)
    const unsigned long long* bits1;
    int B, H, Sq;
    float scale;
    // v_transposed: V0/V1 hold V^T [B, H, Dh, vstride] with keys at vt_pos_f32 (this
    // kernel) or vt_pos_bf16 (launch_attention32); vstride is a multiple of 64 and padding
    // columns hold finite values.
    bool v_transposed;
    int vstride0, vstride1;
    // prescaled: Q already multiplied by scale * log2(e) (the QKV epilogue does this).
    bool prescaled;
    // epilogue: out_mode 0 -> O [B*Sq, H*Dh] (T) = gate[m, h*Dh+d] * attn;
    //           out_mode 1 -> Of [B, H, Sq, Dh] f32
    int out_mode;
    const T* G;
    T* O;
    float* Of;
};
template <typename T, int DH>
int launch_attention(const AttnArgs<T>& a, hipStream_t st);
// bf16, Dh = 64, V^T in vt_pos_bf16 order, Q pre-scaled (kernels_attn32.hip).
int launch_attention32(const AttnArgs<bf16>& a, hipStream_t st);

}  // namespace irodori
