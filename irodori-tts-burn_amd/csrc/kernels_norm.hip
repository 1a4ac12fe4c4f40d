// HBM-bound row kernels: RMSNorm, adaLN modulation, in_proj + modulation, output head.
// One wavefront per row, 4 rows per
// 256-thread workgroup; rows are read with 16-byte loads and reduced in registers with
// cross-lane shuffles (no LDS), so each row is read from HBM exactly once.
#include "common.hpp"
#include "kernels.hpp"

namespace irodori {

namespace {

constexpr int kRowsPerBlock = 4;

__device__ __forceinline__ int mod_vec(const ModTable& mt, int b) {
    return mod_vec_index(mt, mt.step ? *mt.step : 0, b);
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
// D % 4 == 0; each lane owns float4 chunks lane*4 + 256*j.  h (nullable) gets the values in
// the compute dtype; q8 / q8s (nullable, D % 32 == 0) their fp8 GEMM-operand form.
template <typename T, int NCH>
__global__ __launch_bounds__(256) void norm_mod_kernel(const float* __restrict__ x,
                                                       T* __restrict__ h, int M, int S, int D,
                                                       float eps, ModTable mt, int layer,
                                                       int kind, uint8_t* __restrict__ q8,
                                                       uint8_t* __restrict__ q8s) {
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
    // Every chunk's scale / shift loads go out together after the reduction, before the first
    // store (one cache round trip per row, not one per chunk): one straight-line body when D
    // fills the chunks, a guarded one otherwise.
    auto body = [&](auto full_c) {
        constexpr bool FULL = decltype(full_c)::value;
        float4 sc[NCH], sh[NCH];
#pragma unroll
        for (int j = 0; j < NCH; j++) {
            const int d = lane * 4 + 256 * j;
            if (FULL || d < D) {
                sc[j] = *reinterpret_cast<const float4*>(scale + d);
                sh[j] = *reinterpret_cast<const float4*>(shift + d);
            }
        }
#pragma unroll
        for (int j = 0; j < NCH; j++) {
            const int d = lane * 4 + 256 * j;
            if (!FULL && d >= D) break;
            const float h0 = v[j].x / rms * (1.f + sc[j].x) + sh[j].x, h1 = v[j].y / rms * (1.f + sc[j].y) + sh[j].y;
            const float h2 = v[j].z / rms * (1.f + sc[j].z) + sh[j].z, h3 = v[j].w / rms * (1.f + sc[j].w) + sh[j].w;
            if (h) store4<T>(h + (size_t)row * D + d, h0, h1, h2, h3);
            if (q8)
                mx_store4_group8(h0, h1, h2, h3, q8 + (size_t)row * D + d, q8s + (size_t)row * (D / 32) + d / 32,
                                 lane);
        }
    };
    if (D == 256 * NCH) body(std::true_type{});
    else body(std::false_type{});
}

// The fused adaLN's operand of one (layer, kind) from the residual x: h = x (1 + scale)
// in the compute dtype and rstat [M, D/32] the sums of x^2 per 32 columns (the GEMM that
// reads h applies 1 / rms and the shift).  Lane chunks as in norm_mod_kernel: a 32-column
// block is the quads of 8 neighbouring lanes.
template <typename T, int NCH>
__global__ __launch_bounds__(256) void mod_stats_kernel(const float* __restrict__ x, T* __restrict__ h, int M,
                                                        int S, int D, ModTable mt, int layer, int kind,
                                                        float* __restrict__ rstat) {
    int row = blockIdx.x * kRowsPerBlock + threadIdx.x / 64, lane = threadIdx.x % 64;
    if (row >= M) return;
    const float* xr = x + (size_t)row * D;
    const float* scale = mod_base(mt, row / S, layer, kind, D) + D;
#pragma unroll
    for (int j = 0; j < NCH; j++) {
        int d = lane * 4 + 256 * j;
        if (d >= D) break;
        const float4 v = *reinterpret_cast<const float4*>(xr + d);
        const float4 sc = *reinterpret_cast<const float4*>(scale + d);
        store4<T>(h + (size_t)row * D + d, v.x * (1.f + sc.x), v.y * (1.f + sc.y), v.z * (1.f + sc.z),
                  v.w * (1.f + sc.w));
        float q = v.x * v.x + v.y * v.y + v.z * v.z + v.w * v.w;
        q += __shfl_xor(q, 1, 64);
        q += __shfl_xor(q, 2, 64);
        q += __shfl_xor(q, 4, 64);
        if ((lane & 7) == 0) rstat[(size_t)row * (D / 32) + d / 32] = q;
    }
}

// in_proj (x = x_src @ W_in + b_in, dit/model.rs:370) fused with the first adaLN.  A
// 256-thread block owns ROWS rows (8, or 2 when that leaves too few blocks to fill the chip); thread t owns the column quads 4 t + 1024 j (j <
// NCH) of every row, so each W_in quad is loaded once per block and applied to all its
// rows (W_in stays in L2 and is streamed M / ROWS times).  The source rows are staged
// in LDS 64 latent channels at a time; the row RMS reduces over lanes, then over the 4
// wavefronts through LDS.

// With rstat set (the fused adaLN of the bf16 model path) h gets x (1 + scale) instead, and
// rstat [M, D/32] the sums of x^2 per 32 columns (8 neighbouring lanes hold one block).
// copies > 1: the M rows are computed once and every output (x, h, rstat, q8, q8s) is also
// written to the copies - 1 row blocks that follow, M rows apart (batch rows that read the
// same source row and modulation vector).
template <typename T, int NCH, int ROWS>
__global__ __launch_bounds__(256) void inproj_norm_kernel(
    const float* __restrict__ x_src, int src_batches, const float* __restrict__ in_w,
    const float* __restrict__ in_b, float* __restrict__ x, T* __restrict__ h, int M, int S, int P,
    int D, float eps, ModTable mt, uint8_t* __restrict__ q8, uint8_t* __restrict__ q8s,
    float* __restrict__ rstat, int copies) {
    __shared__ float xs[ROWS][64];
    __shared__ float red[ROWS][4];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int row0 = blockIdx.x * ROWS;
    float4 acc[ROWS][NCH];
#pragma unroll
    for (int j = 0; j < NCH; j++) {
        const int d = 4 * tid + 1024 * j;
        const float4 bv = d < D ? *reinterpret_cast<const float4*>(in_b + d) : make_float4(0, 0, 0, 0);
#pragma unroll
        for (int r = 0; r < ROWS; r++) acc[r][j] = bv;
    }
    for (int p0 = 0; p0 < P; p0 += 64) {
        const int pn = P - p0 < 64 ? P - p0 : 64;
        __syncthreads();
        for (int e = tid; e < ROWS * 64; e += 256) {
            const int r = e / 64, pp = e % 64, row = row0 + r;
            float v = 0.f;
            if (row < M && pp < pn) {
                const int b = row / S, sq = row % S;
                v = x_src[((size_t)(b % src_batches) * S + sq) * P + p0 + pp];
            }
            xs[r][pp] = v;
        }
        __syncthreads();
        // 16 W_in quads per column chunk are loaded together so their latencies overlap.
#pragma unroll
        for (int j = 0; j < NCH; j++) {
            const int d = 4 * tid + 1024 * j;
            if (d >= D) break;
            for (int c0 = 0; c0 < pn; c0 += 16) {
                float4 wv[16];
#pragma unroll
                for (int i = 0; i < 16; i++)
                    wv[i] = c0 + i < pn ? *reinterpret_cast<const float4*>(in_w + (size_t)(p0 + c0 + i) * D + d)
                                        : make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
                for (int i = 0; i < 16; i++) {
#pragma unroll
                    for (int r = 0; r < ROWS; r++) {
                        const float a = xs[r][(c0 + i) & 63];
                        acc[r][j].x += a * wv[i].x;
                        acc[r][j].y += a * wv[i].y;
                        acc[r][j].z += a * wv[i].z;
                        acc[r][j].w += a * wv[i].w;
                    }
                }
            }
        }
    }
    // Store x and reduce the per-row sums of squares.
#pragma unroll
    for (int r = 0; r < ROWS; r++) {
        const int row = row0 + r;
        float ss = 0.f;
#pragma unroll
        for (int j = 0; j < NCH; j++) {
            const int d = 4 * tid + 1024 * j;
            if (d >= D) break;
            const float4 v = acc[r][j];
            if (row < M)
                for (int cp = 0; cp < copies; cp++)
                    *reinterpret_cast<float4*>(x + ((size_t)cp * M + row) * D + d) = v;
            float q = v.x * v.x + v.y * v.y + v.z * v.z + v.w * v.w;
            ss += q;
            if (rstat) {
                // Columns 32 c .. 32 c + 31 are the quads of lanes 8 c' .. 8 c' + 7.
                q += __shfl_xor(q, 1, 64);
                q += __shfl_xor(q, 2, 64);
                q += __shfl_xor(q, 4, 64);
                if (row < M && (tid & 7) == 0)
                    for (int cp = 0; cp < copies; cp++)
                        rstat[((size_t)cp * M + row) * (D / 32) + d / 32] = q;
            }
        }
        ss = wave_sum(ss);
        if (lane == 0) red[r][wave] = ss;
    }
    __syncthreads();
    if (rstat) {  // fused adaLN: the GEMMs apply 1 / rms and the shift themselves
#pragma unroll
        for (int r = 0; r < ROWS; r++) {
            const int row = row0 + r;
            if (row >= M) break;
            const float* scale = mod_base(mt, row / S, 0, 0, D) + D;
#pragma unroll
            for (int j = 0; j < NCH; j++) {
                const int d = 4 * tid + 1024 * j;
                if (d >= D) break;
                const float4 sc = *reinterpret_cast<const float4*>(scale + d);
                const float4 v = acc[r][j];
                for (int cp = 0; cp < copies; cp++)
                    store4<T>(h + ((size_t)cp * M + row) * D + d, v.x * (1.f + sc.x), v.y * (1.f + sc.y),
                              v.z * (1.f + sc.z), v.w * (1.f + sc.w));
            }
        }
        return;
    }
#pragma unroll
    for (int r = 0; r < ROWS; r++) {
        const int row = row0 + r;
        if (row >= M) break;
        const float rms = sqrtf((red[r][0] + red[r][1] + red[r][2] + red[r][3]) / (float)D + eps);
        const float* base = mod_base(mt, row / S, 0, 0, D);
        const float* shift = base;
        const float* scale = base + D;
#pragma unroll
        for (int j = 0; j < NCH; j++) {
            const int d = 4 * tid + 1024 * j;
            if (d >= D) break;
            const float4 sc = *reinterpret_cast<const float4*>(scale + d);
            const float4 sh = *reinterpret_cast<const float4*>(shift + d);
            const float4 v = acc[r][j];
            const float h0 = v.x / rms * (1.f + sc.x) + sh.x, h1 = v.y / rms * (1.f + sc.y) + sh.y;
            const float h2 = v.z / rms * (1.f + sc.z) + sh.z, h3 = v.w / rms * (1.f + sc.w) + sh.w;
            for (int cp = 0; cp < copies; cp++) {
                const size_t cr = (size_t)cp * M + row;
                if (h) store4<T>(h + cr * D + d, h0, h1, h2, h3);
                if (q8) mx_store4_group8(h0, h1, h2, h3, q8 + cr * D + d, q8s + cr * (D / 32) + d / 32, lane);
            }
        }
    }
}

// Output head: one 256-thread block per FR latent frames and row group (NR rows;
// blockIdx.y is the group).  v[b,s,p] = (sum_d x[b,s,d] * W'[d,p]) /
// rms(x[b,s,:]) + b_out[p] with W' = out_norm.weight (.) W_out folded at ingest, stored
// [D][PT] with the columns past P zero — the same product as out_proj(out_norm(x))
// (norm.rs:25-39, dit/model.rs:391-392).  The group's rows are staged in LDS; thread
// (kk, q) accumulates the output quad p = 4 q .. 4 q + 3 of every staged row over its own
// KPT = D / KL consecutive k, so one wavefront load covers 64 / QN whole W' rows (coalesced;
// W' is read once per block from L2) and a thread's loads sit at immediate offsets of one
// base.  Staged rows keep 4 pad floats after every 32 (the 64 / QN distinct k of one LDS
// read fall in distinct banks).  The staging loads, the first KB W' quads of each thread and
// the sampler state the update reads are all issued before the first LDS write, so their
// latencies overlap.  The KL partial sums reduce across lanes, then across the 4 wavefronts through
// LDS.  Plain head: groups are consecutive rows.  Sampler
// evaluation: group u holds the active roles' rows of utterance u, and the block applies
// the guided combine and the integrator update to them (euler_sampler.rs:460-467,
// :497-510, :683-714) — one kernel after the role chains join.  With rf.advance set the
// last workgroup to finish also advances the step counter (every workgroup has read it by
// then).  Role and plan arrays are indexed by unrolled selects only (a runtime index would
// place them in scratch).
template <int PT, int NR, int FR>
__global__ __launch_bounds__(256) void final_kernel(FinalArgs a) {
    constexpr int QN = PT / 4;    // output quads per W' row
    constexpr int KL = 256 / QN;  // k positions per pass of the block
    constexpr int R = NR * FR;    // staged row slot f * NR + i
    // W' quads in flight per thread (offsets below 4 KB; all of them for D = 1024, PT = 32)
    constexpr int KB = PT == 32 ? 32 : (PT == 64 ? 16 : (PT == 128 ? 8 : 4));
    static_assert(FR * PT <= 256, "one update element per thread");
    extern __shared__ __attribute__((aligned(16))) float fsm[];
    const int D = a.D, P = a.P;
    const int DP = D + D / 8;        // staged row stride (4 pad floats per 32)
    const int KPT = D / KL;          // D % KL == 0
    float* xs = fsm;                 // [R][DP]
    float* red = xs + R * DP;        // [4][R][PT]
    float* vals = red + 4 * R * PT;  // [R][PT]
    float* rinv = vals + R * PT;     // [R]
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int q = tid % QN, kk = tid / QN;
    const int s0 = blockIdx.x * FR;
    const int nf = a.S - s0 < FR ? a.S - s0 : FR;
    const bool rf = a.rf.plan != nullptr;
    int step = 0;
    RfEval ev{};
    if (rf) {
        step = *a.rf.step;
        ev = a.rf.plan[2 * step + a.rf.phase];
    }
    // One row group per blockIdx.y: the launcher's grid.y is the group count (at most the
    // context's row limit, 65535).
    const int g = blockIdx.y;
    // Row of slot i: the group's i-th row (a plain head's short last group repeats its
    // first row).
    auto row_of = [&](int i) {
        if (rf) {
            int ro = a.role[0];
#pragma unroll
            for (int k = 1; k < NR; k++)
                if (i == k) ro = a.role[k];
            return ro * a.B + g;
        }
        const int b = g * NR + i;
        return b < a.B ? b : g * NR;
    };
    // Staged rows [R][D]: float4 j of chunk c of this thread is element 4 ((c SC + j) 256 +
    // tid); frames past S read frame nf - 1 and stage zeros.  One chunk holds every element
    // for D = 1024; it is issued before the W' quads so that both latencies overlap, and its
    // loads are all in flight before the first LDS write waits on them.
    constexpr int SC = R;
    const int nst = R * D / 4;  // D % 4 == 0
    float4 sv[SC];
    auto stage_issue = [&](int c) {
#pragma unroll
        for (int j = 0; j < SC; j++) {
            const int idx = (c * SC + j) * 256 + tid;
            const int e = (idx < nst ? idx : 0) * 4;
            const int r = e / D, d = e - r * D, f = r / NR, i = r - f * NR;
            sv[j] = *reinterpret_cast<const float4*>(
                a.x + ((size_t)row_of(i) * a.S + s0 + (f < nf ? f : nf - 1)) * D + d);
        }
    };
    auto stage_write = [&](int c) {
#pragma unroll
        for (int j = 0; j < SC; j++) {
            const int idx = (c * SC + j) * 256 + tid;
            if (idx < nst) {
                const int e = idx * 4, r = e / D, d = e - r * D;
                const float4 v = r / NR < nf ? sv[j] : make_float4(0.f, 0.f, 0.f, 0.f);
                *reinterpret_cast<float4*>(xs + r * DP + d + 4 * (d >> 5)) = v;
            }
        }
    };
    stage_issue(0);
    // The first KB W' quads of this thread (rows past D, when KPT < KB, re-read row D - 1
    // and go unused: the k loop below then loads its rows itself).
    const int kb0 = kk * KPT;
    const float* wq = a.out_w + (size_t)kb0 * PT + 4 * q;
    float4 w[KB];
#pragma unroll
    for (int i = 0; i < KB; i++)
        w[i] = *reinterpret_cast<const float4*>(wq + (size_t)(kb0 + i < D ? i : D - 1 - kb0) * PT);
    // Sampler state element of this thread's update (thread e < nf * PT: frame e / PT,
    // column e % PT; other threads read an element in range and leave it unused).
    float xst = 0.f;
    if (rf) {
        const int fe = tid / PT < nf ? tid / PT : nf - 1, pe = tid % PT < P ? tid % PT : P - 1;
        xst = a.rf.x[(g * a.S + s0 + fe) * P + pe];
    }
    stage_write(0);
    for (int c = 1; c * SC * 256 < nst; c++) {
        stage_issue(c);
        stage_write(c);
    }
    __syncthreads();
    for (int r = wave; r < R; r += 4) {
        float ss = 0.f;
        for (int d = lane; d < D; d += 64) {
            const float xv = xs[r * DP + d + 4 * (d >> 5)];
            ss += xv * xv;
        }
        ss = wave_sum(ss);
        if (lane == 0) rinv[r] = 1.f / sqrtf(ss / (float)D + a.eps);
    }
    float4 acc[R];
#pragma unroll
    for (int r = 0; r < R; r++) acc[r] = make_float4(0.f, 0.f, 0.f, 0.f);
    auto fma_k = [&](int k, const float4& wv) {  // k: row of W' and column of the staged rows
        const int kx = k + 4 * (k >> 5);
#pragma unroll
        for (int r = 0; r < R; r++) {
            const float xv = xs[r * DP + kx];
            acc[r].x += xv * wv.x;
            acc[r].y += xv * wv.y;
            acc[r].z += xv * wv.z;
            acc[r].w += xv * wv.w;
        }
    };
    int k0 = 0;
    for (; k0 + KB <= KPT; k0 += KB) {
        if (k0 > 0) {
#pragma unroll
            for (int i = 0; i < KB; i++) w[i] = *reinterpret_cast<const float4*>(wq + (size_t)(k0 + i) * PT);
        }
#pragma unroll
        for (int i = 0; i < KB; i++) fma_k(kb0 + k0 + i, w[i]);
    }
    for (; k0 < KPT; k0++) fma_k(kb0 + k0, *reinterpret_cast<const float4*>(wq + (size_t)k0 * PT));
    // Lanes q, q + QN, ... of a wavefront hold one quad's partial sums.
#pragma unroll
    for (int r = 0; r < R; r++) {
        float4 v = acc[r];
#pragma unroll
        for (int m = QN; m < 64; m <<= 1) {
            v.x += __shfl_xor(v.x, m, 64);
            v.y += __shfl_xor(v.y, m, 64);
            v.z += __shfl_xor(v.z, m, 64);
            v.w += __shfl_xor(v.w, m, 64);
        }
        if (lane < QN) *reinterpret_cast<float4*>(red + (wave * R + r) * PT + 4 * q) = v;
    }
    __syncthreads();
    for (int idx = tid; idx < R * PT; idx += 256) {  // R * PT may exceed the block
        const int r = idx / PT, pp = idx % PT;
        const float v = red[r * PT + pp] + red[(R + r) * PT + pp] + red[(2 * R + r) * PT + pp] +
                        red[(3 * R + r) * PT + pp];
        vals[r * PT + pp] = pp < P ? v * rinv[r] + a.out_b[pp] : 0.f;
    }
    __syncthreads();
    for (int e = tid; e < nf * PT; e += 256) {  // nf * PT <= 256: one pass
        const int f = e / PT, pp = e % PT, sq = s0 + f;
        if (pp >= P) continue;
        if (!rf) {
#pragma unroll
            for (int i = 0; i < NR; i++)
                if (g * NR + i < a.B) a.v_out[((size_t)(g * NR + i) * a.S + sq) * P + pp] = vals[(f * NR + i) * PT + pp];
            continue;
        }
        const float v0 = vals[(f * NR) * PT + pp];
        float v = v0;
#pragma unroll
        for (int k = 0; k < 3; k++) {
            if (k >= ev.nterm) break;
            int slot = 0;
#pragma unroll
            for (int i = 1; i < NR; i++)
                if (a.role[i] == ev.role[k]) slot = i;
            v = v + (v0 - vals[(f * NR + slot) * PT + pp]) * ev.scale[k];
        }
        rf_apply(a.rf, ev, step, (g * a.S + sq) * P + pp, v, xst);
    }
    if (rf && a.rf.advance) {
        __syncthreads();
        if (tid == 0) {
            const int total = gridDim.x * gridDim.y;
            if (atomicAdd(a.rf.done, 1) == total - 1) {
                *a.rf.done = 0;
                *a.rf.step = step + 1;
            }
        }
    }
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
                     int layer, int kind, hipStream_t st, uint8_t* q8, uint8_t* q8s) {
    int grid = (M + kRowsPerBlock - 1) / kRowsPerBlock;
    int nch = (D + 255) / 256;
    if (nch <= 1)
        norm_mod_kernel<T, 1><<<grid, 256, 0, st>>>(x, h, M, S, D, eps, mt, layer, kind, q8, q8s);
    else if (nch <= 2)
        norm_mod_kernel<T, 2><<<grid, 256, 0, st>>>(x, h, M, S, D, eps, mt, layer, kind, q8, q8s);
    else if (nch <= 4)
        norm_mod_kernel<T, 4><<<grid, 256, 0, st>>>(x, h, M, S, D, eps, mt, layer, kind, q8, q8s);
    else if (nch <= 8)
        norm_mod_kernel<T, 8><<<grid, 256, 0, st>>>(x, h, M, S, D, eps, mt, layer, kind, q8, q8s);
    else
        norm_mod_kernel<T, 16><<<grid, 256, 0, st>>>(x, h, M, S, D, eps, mt, layer, kind, q8, q8s);
}

template <typename T>
void launch_mod_stats(const float* x, T* h, int M, int S, int D, ModTable mt, int layer, int kind, float* rstat,
                      hipStream_t st) {
    int grid = (M + kRowsPerBlock - 1) / kRowsPerBlock;
    int nch = (D + 255) / 256;
    if (nch <= 1) mod_stats_kernel<T, 1><<<grid, 256, 0, st>>>(x, h, M, S, D, mt, layer, kind, rstat);
    else if (nch <= 2) mod_stats_kernel<T, 2><<<grid, 256, 0, st>>>(x, h, M, S, D, mt, layer, kind, rstat);
    else if (nch <= 4) mod_stats_kernel<T, 4><<<grid, 256, 0, st>>>(x, h, M, S, D, mt, layer, kind, rstat);
    else if (nch <= 8) mod_stats_kernel<T, 8><<<grid, 256, 0, st>>>(x, h, M, S, D, mt, layer, kind, rstat);
    else mod_stats_kernel<T, 16><<<grid, 256, 0, st>>>(x, h, M, S, D, mt, layer, kind, rstat);
}
template void launch_mod_stats<bf16>(const float*, bf16*, int, int, int, ModTable, int, int, float*, hipStream_t);

template <typename T>
void launch_inproj_norm(const float* x_src, int src_batches, const float* in_w,
                        const float* in_b, float* x, T* h, int M, int S, int P, int D, float eps,
                        ModTable mt, hipStream_t st, uint8_t* q8, uint8_t* q8s, float* rstat, int copies) {
    const int nch = (D + 1023) / 1024;
    const bool fine = (M + 7) / 8 < 512;  // fewer than two blocks per CU at 8 rows
    const int rows = fine ? 2 : 8, grid = (M + rows - 1) / rows;
#define IRO_INPROJ(N, R)                                                                      \
    inproj_norm_kernel<T, N, R><<<grid, 256, 0, st>>>(x_src, src_batches, in_w, in_b, x, h, M, \
                                                      S, P, D, eps, mt, q8, q8s, rstat, copies)
    if (fine) {
        if (nch <= 1) IRO_INPROJ(1, 2);
        else if (nch <= 2) IRO_INPROJ(2, 2);
        else IRO_INPROJ(4, 2);
    } else {
        if (nch <= 1) IRO_INPROJ(1, 8);
        else if (nch <= 2) IRO_INPROJ(2, 8);
        else IRO_INPROJ(4, 8);
    }
#undef IRO_INPROJ
}

template void launch_norm_mod<float>(const float*, float*, int, int, int, float, ModTable, int,
                                     int, hipStream_t, uint8_t*, uint8_t*);
template void launch_norm_mod<bf16>(const float*, bf16*, int, int, int, float, ModTable, int,
                                    int, hipStream_t, uint8_t*, uint8_t*);
template void launch_inproj_norm<float>(const float*, int, const float*, const float*, float*,
                                        float*, int, int, int, int, float, ModTable,
                                        hipStream_t, uint8_t*, uint8_t*, float*, int);
template void launch_inproj_norm<bf16>(const float*, int, const float*, const float*, float*,
                                       bf16*, int, int, int, int, float, ModTable, hipStream_t,
                                       uint8_t*, uint8_t*, float*, int);

template <int PT, int NR, int FR>
static void launch_final_cfg(const FinalArgs& a, hipStream_t st) {
    constexpr int R = NR * FR;
    const size_t lds = sizeof(float) * ((size_t)R * (a.D + a.D / 8) + (size_t)4 * R * PT + (size_t)R * PT + R);
    // Sized for the widest model the instantiation serves: D <= 4096 with at most 6 staged
    // rows (the launcher keeps wider models there), D <= 2048 otherwise.
    constexpr int kMaxD = R <= 6 ? 4096 : 2048;
    constexpr int kMax = (int)sizeof(float) * (R * (kMaxD + kMaxD / 8) + 4 * R * PT + R * PT + R);
    static_assert(kMax <= 160 * 1024, "staged rows fit the LDS");
    static LdsLimit lds_limit;
    (void)set_lds_limit_once(lds_limit, (const void*)final_kernel<PT, NR, FR>, kMax);
    const int ngroups = a.rf.plan ? a.B : (a.B + NR - 1) / NR;  // <= 65535 (row limit)
    const dim3 grid((a.S + FR - 1) / FR, ngroups);
    final_kernel<PT, NR, FR><<<grid, 256, lds, st>>>(a);
}

// Four, two or one frames per block: the most that still gives 256 blocks (each block reads
// all of W' from L2, so coarser blocks win once there are enough of them).
template <int PT, int FR>
static void launch_final_fr(const FinalArgs& a, hipStream_t st) {
    const int nr = a.rf.plan ? a.nrole : 2;
    if (nr <= 1) launch_final_cfg<PT, 1, FR>(a, st);
    else if (nr == 2) launch_final_cfg<PT, 2, FR>(a, st);
    else launch_final_cfg<PT, 3, FR>(a, st);
}
template <int PT>
static void launch_final_pt(const FinalArgs& a, hipStream_t st) {
    const int nr = a.rf.plan ? a.nrole : 2;
    const int ngroups = a.rf.plan ? a.B : (a.B + nr - 1) / nr;
    // One update element per thread: PT = 128 takes at most two frames per block, 256 one.
    // Models wider than 2048 stage at most 6 rows (two frames of three roles).
    if constexpr (PT * 4 <= 256) {
        if (a.D <= 2048 && (long)((a.S + 3) / 4) * ngroups >= 256) {
            launch_final_fr<PT, 4>(a, st);
            return;
        }
    }
    if constexpr (PT * 2 <= 256) {
        if ((long)((a.S + 1) / 2) * ngroups >= 256) {
            launch_final_fr<PT, 2>(a, st);
            return;
        }
    }
    launch_final_fr<PT, 1>(a, st);
}

void launch_final(const FinalArgs& a, hipStream_t st) {
    if (a.P <= 32) launch_final_pt<32>(a, st);
    else if (a.P <= 64) launch_final_pt<64>(a, st);
    else if (a.P <= 128) launch_final_pt<128>(a, st);
    else launch_final_pt<256>(a, st);
}


void launch_scale_copy(const float* src, float* dst, int n, float s, hipStream_t st) {
    scale_copy_kernel<<<(n + 255) / 256, 256, 0, st>>>(src, dst, n, s);
}

}  // namespace irodori
