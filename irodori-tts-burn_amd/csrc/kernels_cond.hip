// Timestep conditioning: sinusoidal embedding, cond_module MLP and the low-rank adaLN
// projections.  These depend only on t, so for an RF run they are evaluated for every
// step of the schedule at once (a handful of launches at the start of the run) and the
// per-step kernels index the resulting table by a device step counter.  Arithmetic is
// f32 throughout (the modulation vectors scale every activation of the block).
#include "common.hpp"
#include "kernels.hpp"

namespace irodori {

namespace {

// rope.rs:141-165: emb = [cos(t f_i) | sin(t f_i)], f_i = 1000 exp(-ln(1e4) i / half).
__global__ void timestep_embedding_kernel(const float* __restrict__ t, int nvec, int t_dim,
                                          float* __restrict__ out) {
    int v = blockIdx.y, i = blockIdx.x * blockDim.x + threadIdx.x;
    int half = t_dim / 2;
    if (v >= nvec || i >= half) return;
    float f = 1000.0f * expf((-logf(10000.0f) * (float)i) / (float)half);
    float a = t[v] * f;
    out[(size_t)v * t_dim + i] = cosf(a);
    out[(size_t)v * t_dim + half + i] = sinf(a);
}

constexpr int kKTile = 64;  // staged X columns per pass

__device__ __forceinline__ float apply_act(float v, int act) {
    if (act == 1) return silu_f(v);
    if (act == 2) return tanhf(v);
    return v;
}

// Y[v, n] = act_out(act_in(X[v, :]) @ W[:, n] + bias[n] + R[v, n]) for every job
// (blockIdx.y), COLS-column block (blockIdx.x) and VC-vector chunk (blockIdx.z).  The 256
// threads are COLS columns x KG = 256 / COLS k-groups: thread (kg, c) owns column
// n = COLS blockIdx.x + c and the k values k = kg (mod KG), accumulating all VC vectors of
// the chunk in registers, so W is streamed once per vector chunk (a wavefront reads 64 / COLS
// row segments of COLS consecutive columns per k).  K advances in tiles of 64: the X tile
// (activation applied) is staged transposed in LDS (one k = VC vectors, broadcast 16-byte
// reads), and the W and X values of tile t + 1 are loaded into registers while tile t is
// computed.  The k-groups are summed through LDS at the end, in k-group order.
template <int VC, int COLS>
__global__ __launch_bounds__(256) void vec_linear_kernel(const VecLinJob* __restrict__ jobs, int nvec) {
    constexpr int KG = 256 / COLS, NK = kKTile / KG, NX = VC * kKTile / 256;
    static_assert(VC % 4 == 0 && KG * COLS == 256 && NX * 256 == VC * kKTile, "tile shapes");
    __shared__ __attribute__((aligned(16))) float xs[kKTile][VC];
    __shared__ float red[KG - 1][VC][COLS];
    const VecLinJob jb = jobs[blockIdx.y];
    if (blockIdx.x * COLS >= jb.N) return;  // uniform: this job has fewer columns
    const int c = threadIdx.x % COLS, kg = threadIdx.x / COLS;
    const int n = blockIdx.x * COLS + c;
    const bool active = n < jb.N;
    const int v0 = blockIdx.z * VC;
    const int nv = nvec - v0 < VC ? nvec - v0 : VC;
    float acc[VC];
#pragma unroll
    for (int v = 0; v < VC; v++) acc[v] = 0.f;
    float wv[NK], xv[NX];
    auto load_tile = [&](int k0) {
        const int kt = jb.K - k0 < kKTile ? jb.K - k0 : kKTile;
#pragma unroll
        for (int i = 0; i < NK; i++) {
            const int k = kg + KG * i;
            wv[i] = active && k < kt ? jb.W[(size_t)(k0 + k) * jb.N + n] : 0.f;
        }
#pragma unroll
        for (int i = 0; i < NX; i++) {
            const int e = threadIdx.x + 256 * i, v = e % VC, k = e / VC;  // conflict-free LDS writes
            xv[i] = v < nv && k < kt ? jb.X[(size_t)(v0 + v) * jb.ldx + k0 + k] : 0.f;
        }
    };
    load_tile(0);
    for (int k0 = 0; k0 < jb.K; k0 += kKTile) {
        __syncthreads();  // every thread is past the previous tile's X reads
#pragma unroll
        for (int i = 0; i < NX; i++) {
            const int e = threadIdx.x + 256 * i;
            xs[e / VC][e % VC] = apply_act(xv[i], jb.act_in);
        }
        float wc[NK];
#pragma unroll
        for (int i = 0; i < NK; i++) wc[i] = wv[i];
        __syncthreads();
        if (k0 + kKTile < jb.K) load_tile(k0 + kKTile);  // in flight during this tile
        if (active) {
            const int kt = jb.K - k0 < kKTile ? jb.K - k0 : kKTile;
#pragma unroll
            for (int i = 0; i < NK; i++) {
                const int k = kg + KG * i;
                if (k >= kt) break;
                const float4* xr = reinterpret_cast<const float4*>(&xs[k][0]);
#pragma unroll
                for (int q = 0; q < VC / 4; q++) {
                    const float4 x4 = xr[q];
                    acc[4 * q] += x4.x * wc[i];
                    acc[4 * q + 1] += x4.y * wc[i];
                    acc[4 * q + 2] += x4.z * wc[i];
                    acc[4 * q + 3] += x4.w * wc[i];
                }
            }
        }
    }
    if (kg > 0) {
#pragma unroll
        for (int v = 0; v < VC; v++) red[kg - 1][v][c] = acc[v];
    }
    __syncthreads();
    if (kg == 0 && active) {
        for (int v = 0; v < nv; v++) {
            float y = acc[v];
#pragma unroll
            for (int g2 = 0; g2 < KG - 1; g2++) y += red[g2][v][c];
            if (jb.bias) y += jb.bias[n];
            if (jb.R) y += jb.R[(size_t)(v0 + v) * jb.ldr + n];
            jb.Y[(size_t)(v0 + v) * jb.ldy + n] = apply_act(y, jb.act_out);
        }
    }
}

template <int VC, int COLS>
void launch_vec_linear_cfg(const VecLinJob* d_jobs, int njobs, int nvec, int max_n, hipStream_t st) {
    dim3 grid((max_n + COLS - 1) / COLS, njobs, (nvec + VC - 1) / VC);
    vec_linear_kernel<VC, COLS><<<grid, 256, 0, st>>>(d_jobs, nvec);
}

// Shift rows of the modulation table [vec][layer][kind][chunk][D] as bf16 GEMM operands:
// block (v, l * 2 + k) copies chunk 0 of (v, l, k) to stage row (l * 2 + k) * cap + v.
__global__ __launch_bounds__(256) void shift_stage_kernel(const float* __restrict__ tab, int cap, int L, int D,
                                                          bf16* __restrict__ stage) {
    const int v = blockIdx.x, lk = blockIdx.y;
    const float* src = tab + ((size_t)v * L * 6 + (size_t)lk * 3) * D;
    bf16* dst = stage + ((size_t)lk * cap + v) * D;
    for (int d = threadIdx.x; d < D; d += 256) dst[d] = static_cast<bf16>(src[d]);
}

}  // namespace

void launch_shift_stage(const float* tab, int nvec, int cap, int L, int D, bf16* stage, hipStream_t st) {
    shift_stage_kernel<<<dim3(nvec, 2 * L), 256, 0, st>>>(tab, cap, L, D, stage);
}

void launch_timestep_embedding(const float* t, int nvec, int t_dim, float* out, hipStream_t st) {
    dim3 grid((t_dim / 2 + 255) / 256, nvec);
    timestep_embedding_kernel<<<grid, 256, 0, st>>>(t, nvec, t_dim, out);
}

// Vector chunks of 16 (an RF run's 41 timesteps are three chunks, run side by side).
// Columns: 64 per block when the jobs x column blocks fill the chip, else 16 per block with
// 16 k-groups (the cond MLP's single-job launches).
void launch_vec_linear(const VecLinJob* d_jobs, int njobs, int nvec, int max_n, hipStream_t st) {
    if ((long)((max_n + 63) / 64) * njobs >= 256) launch_vec_linear_cfg<16, 64>(d_jobs, njobs, nvec, max_n, st);
    else launch_vec_linear_cfg<16, 16>(d_jobs, njobs, nvec, max_n, st);
}

}  // namespace irodori
