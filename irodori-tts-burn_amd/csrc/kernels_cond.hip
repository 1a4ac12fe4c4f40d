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

constexpr int kVecChunk = 32;  // vectors per workgroup (blockIdx.z chunks the rest)
constexpr int kCols = 64;      // output columns per workgroup
constexpr int kKGroups = 4;    // k-slices per workgroup, reduced through LDS
constexpr int kKTile = 256;    // staged X columns per pass

__device__ __forceinline__ float apply_act(float v, int act) {
    if (act == 1) return silu_f(v);
    if (act == 2) return tanhf(v);
    return v;
}

// Y[v, n] = act_out(act_in(X[v, :]) @ W[:, n] + bias[n] + R[v, n]) for every job
// (blockIdx.y), 64-column block (blockIdx.x) and 32-vector chunk (blockIdx.z).  Thread
// (kg, c) owns column n = 64 blockIdx.x + c and the k-slice k = kg (mod 4), accumulating
// all vectors of the chunk in registers; a wavefront reads one 256-byte row segment of
// W per k, so W is streamed once per vector chunk.  The X tile (activation applied) is
// staged in LDS and the 4 k-slices are summed through LDS at the end.
__global__ __launch_bounds__(256) void vec_linear_kernel(const VecLinJob* __restrict__ jobs,
                                                         int nvec) {
    __shared__ __attribute__((aligned(16))) float xs[kKTile][kVecChunk];  // transposed: one k = 32 vectors
    __shared__ float red[kKGroups - 1][kVecChunk][kCols];
    const VecLinJob jb = jobs[blockIdx.y];
    if (blockIdx.x * kCols >= jb.N) return;  // uniform: this job has fewer columns
    const int c = threadIdx.x % kCols, kg = threadIdx.x / kCols;
    const int n = blockIdx.x * kCols + c;
    const bool active = n < jb.N;
    const int v0 = blockIdx.z * kVecChunk;
    const int nv = nvec - v0 < kVecChunk ? nvec - v0 : kVecChunk;
    float acc[kVecChunk];
#pragma unroll
    for (int v = 0; v < kVecChunk; v++) acc[v] = 0.f;
    for (int k0 = 0; k0 < jb.K; k0 += kKTile) {
        const int kt = jb.K - k0 < kKTile ? jb.K - k0 : kKTile;
        __syncthreads();
        for (int e = threadIdx.x; e < kVecChunk * kKTile; e += 256) {
            const int v = e % kVecChunk, k = e / kVecChunk;  // conflict-free LDS writes
            float val = 0.f;
            if (v < nv && k < kt) val = apply_act(jb.X[(size_t)(v0 + v) * jb.ldx + k0 + k], jb.act_in);
            xs[k][v] = val;
        }
        __syncthreads();
        if (active) {
            // 16 W values (k = kg, kg + 4, ...) are loaded together so their latencies
            // overlap; each k's 32 vector values are 8 broadcast 16-byte LDS reads.
            for (int kb = 0; kb < kt; kb += 16 * kKGroups) {
                float wv[16];
#pragma unroll
                for (int i = 0; i < 16; i++) {
                    const int k = kb + kg + kKGroups * i;
                    wv[i] = k < kt ? jb.W[(size_t)(k0 + k) * jb.N + n] : 0.f;
                }
#pragma unroll
                for (int i = 0; i < 16; i++) {
                    const int k = kb + kg + kKGroups * i;
                    if (k >= kt) break;
                    const float4* xr = reinterpret_cast<const float4*>(&xs[k][0]);
#pragma unroll
                    for (int q = 0; q < kVecChunk / 4; q++) {
                        const float4 xv = xr[q];
                        acc[4 * q] += xv.x * wv[i];
                        acc[4 * q + 1] += xv.y * wv[i];
                        acc[4 * q + 2] += xv.z * wv[i];
                        acc[4 * q + 3] += xv.w * wv[i];
                    }
                }
            }
        }
    }
    if (kg > 0) {
#pragma unroll
        for (int v = 0; v < kVecChunk; v++) red[kg - 1][v][c] = acc[v];
    }
    __syncthreads();
    if (kg == 0 && active) {
        for (int v = 0; v < nv; v++) {
            float y = acc[v] + red[0][v][c] + red[1][v][c] + red[2][v][c];
            if (jb.bias) y += jb.bias[n];
            if (jb.R) y += jb.R[(size_t)(v0 + v) * jb.ldr + n];
            jb.Y[(size_t)(v0 + v) * jb.ldy + n] = apply_act(y, jb.act_out);
        }
    }
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

void launch_vec_linear(const VecLinJob* d_jobs, int njobs, int nvec, int max_n, hipStream_t st) {
    dim3 grid((max_n + kCols - 1) / kCols, njobs, (nvec + kVecChunk - 1) / kVecChunk);
    vec_linear_kernel<<<grid, 256, 0, st>>>(d_jobs, nvec);
}

}  // namespace irodori
