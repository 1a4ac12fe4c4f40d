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

constexpr int kVecChunk = 32;  // vectors accumulated per thread per pass
constexpr int kKTile = 64;

__device__ __forceinline__ float apply_act(float v, int act) {
    if (act == 1) return silu_f(v);
    if (act == 2) return tanhf(v);
    return v;
}

// Y[v, n] = act_out(act_in(X[v, :]) @ W[:, n] + bias[n] + R[v, n]) for every job
// (blockIdx.y) and column block (blockIdx.x).  Each thread owns one column n and
// accumulates up to kVecChunk vectors, so W (the dominant traffic) is streamed once per
// kVecChunk vectors with coalesced row reads; the X tile is staged in LDS.
__global__ __launch_bounds__(256) void vec_linear_kernel(const VecLinJob* __restrict__ jobs,
                                                         int nvec) {
    __shared__ float xs[kVecChunk][kKTile];
    const VecLinJob jb = jobs[blockIdx.y];
    int n = blockIdx.x * 256 + threadIdx.x;
    bool active = n < jb.N;
    for (int v0 = 0; v0 < nvec; v0 += kVecChunk) {
        int nv = nvec - v0 < kVecChunk ? nvec - v0 : kVecChunk;
        float acc[kVecChunk];
#pragma unroll
        for (int v = 0; v < kVecChunk; v++) acc[v] = 0.f;
        for (int k0 = 0; k0 < jb.K; k0 += kKTile) {
            int kt = jb.K - k0 < kKTile ? jb.K - k0 : kKTile;
            __syncthreads();
            for (int e = threadIdx.x; e < kVecChunk * kKTile; e += 256) {
                int v = e / kKTile, k = e % kKTile;
                float val = 0.f;
                if (v < nv && k < kt) val = apply_act(jb.X[(size_t)(v0 + v) * jb.ldx + k0 + k], jb.act_in);
                xs[v][k] = val;
            }
            __syncthreads();
            if (active) {
                for (int k = 0; k < kt; k++) {
                    float w = jb.W[(size_t)(k0 + k) * jb.N + n];
#pragma unroll
                    for (int v = 0; v < kVecChunk; v++) acc[v] += xs[v][k] * w;
                }
            }
        }
        if (active) {
            for (int v = 0; v < nv; v++) {
                float y = acc[v];
                if (jb.bias) y += jb.bias[n];
                if (jb.R) y += jb.R[(size_t)(v0 + v) * jb.ldr + n];
                jb.Y[(size_t)(v0 + v) * jb.ldy + n] = apply_act(y, jb.act_out);
            }
        }
    }
}

}  // namespace

void launch_timestep_embedding(const float* t, int nvec, int t_dim, float* out, hipStream_t st) {
    dim3 grid((t_dim / 2 + 255) / 256, nvec);
    timestep_embedding_kernel<<<grid, 256, 0, st>>>(t, nvec, t_dim, out);
}

void launch_vec_linear(const VecLinJob* d_jobs, int njobs, int nvec, int max_n, hipStream_t st) {
    dim3 grid((max_n + 255) / 256, njobs);
    vec_linear_kernel<<<grid, 256, 0, st>>>(d_jobs, nvec);
}

}  // namespace irodori
