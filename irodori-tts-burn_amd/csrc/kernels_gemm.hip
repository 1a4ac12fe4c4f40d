// Matrix-core GEMM for the DiT projections: C[M,N] = A[M,K] @ W[N,K]^T with fused
// epilogues.  Both operands are K-contiguous in HBM (weights are re-laid out at ingest).
//
// Data path (gfx950):
//   * K advances in 128-byte slices (64 bf16 / 32 f32 per row).  Each slice of the A and
//     W tiles moves HBM/L2 -> LDS with global_load_lds_dwordx4 (no VGPR staging): one
//     wave instruction fills 8 rows x 128 B, and STAGES slices are in flight.
//   * LDS rows are unpadded; the 16-byte chunk c of row r is stored at c ^ ((r >> 1) & 7),
//     which makes the 32-row fragment reads conflict-free (two 128-byte rows share a
//     256-byte bank line, so rows 2p and 2p+1 use the same xor key).
//   * v_mfma_f32_32x32x16_bf16 (the full-rate bf16 shape on gfx950; 16x16x32 issues at
//     half rate) on 32x32 blocks; the f32 path uses v_mfma_f32_32x32x2_f32 on the same
//     fragments.  4 wavefronts per workgroup in a 2x2 grid.
//   * Workgroup barriers are raw s_barrier after an explicit vmcnt wait for the slice
//     being consumed, so later slices stay in flight across the barrier.
//
// Epilogues (all in registers, no extra pass over HBM):
//   EPI_STORE  C f32
//   EPI_RESID  x += gate * C            (gated residual, diffusion.rs:98 / :104)
//   EPI_SWIGLU U = silu(C1) * C3        (feed_forward.rs:80-84; W rows interleaved per 32)
//   EPI_QKVG   q,k: head RMSNorm (norm.rs:60-74) + half RoPE (rope.rs:82-135);
//              q pre-scaled by Dh^-1/2 log2(e) for the attention softmax;
//              v: scatter to V^T [B,H,Dh,S'] (key-permuted); gate: sigmoid (attention.rs:423)
#include "common.hpp"
#include "kernels.hpp"

namespace irodori {

namespace {

typedef float f32x16 __attribute__((ext_vector_type(16)));

template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}
// Workgroup barrier without the implied memory fence (which would drain every in-flight
// load, including the prefetched slices).
__device__ __forceinline__ void raw_barrier() { asm volatile("s_barrier" ::: "memory"); }

// 16 bytes per lane from global memory straight into LDS (lane i lands at lds + 16 i).
__device__ __forceinline__ void load_lds16(const void* g, void* lds) {
    __builtin_amdgcn_global_load_lds(g, (__attribute__((address_space(3))) void*)lds, 16, 0, 0);
}

__device__ __forceinline__ int swz(int r, int c) { return c ^ ((r >> 1) & 7); }

// One k16 step of a 32x32 block product: bf16 -> one MFMA, f32 -> eight 32x32x2 MFMAs.
// Fragment = the 8 reduction elements a lane supplies (k = 8*(lane/32) + e).
template <typename T>
struct Frag32;
template <>
struct Frag32<bf16> {
    bf16x8 v;
};
template <>
struct Frag32<float> {
    f32x8 v;
};
__device__ __forceinline__ void mma32(f32x16& acc, const Frag32<bf16>& a, const Frag32<bf16>& b) {
    acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a.v, b.v, acc, 0, 0, 0);
}
__device__ __forceinline__ void mma32(f32x16& acc, const Frag32<float>& a, const Frag32<float>& b) {
#pragma unroll
    for (int e = 0; e < 8; e++) acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a.v[e], b.v[e], acc, 0, 0, 0);
}

// Read the fragment of k16 step ks for stage row r (128-byte swizzled rows).
template <typename T>
__device__ __forceinline__ Frag32<T> read_frag(const unsigned char* st, int r, int ks, int h);
template <>
__device__ __forceinline__ Frag32<bf16> read_frag<bf16>(const unsigned char* st, int r, int ks, int h) {
    Frag32<bf16> f;
    f.v = *reinterpret_cast<const bf16x8*>(st + r * 128 + (swz(r, 2 * ks + h) << 4));
    return f;
}
template <>
__device__ __forceinline__ Frag32<float> read_frag<float>(const unsigned char* st, int r, int ks, int h) {
    Frag32<float> f;
    float4 lo = *reinterpret_cast<const float4*>(st + r * 128 + (swz(r, 4 * ks + 2 * h) << 4));
    float4 hi = *reinterpret_cast<const float4*>(st + r * 128 + (swz(r, 4 * ks + 2 * h + 1) << 4));
    f.v[0] = lo.x; f.v[1] = lo.y; f.v[2] = lo.z; f.v[3] = lo.w;
    f.v[4] = hi.x; f.v[5] = hi.y; f.v[6] = hi.z; f.v[7] = hi.w;
    return f;
}

__device__ __forceinline__ const float* gate_vec(const ModTable& mt, int b, int layer, int kind,
                                                int D) {
    int step = mt.step ? *mt.step : 0;
    int vec = step * mt.step_stride + b / mt.rows_per_vec;
    return mt.tab + ((size_t)vec * mt.layers * 6 + (size_t)layer * 6 + kind * 3 + 2) * D;
}

template <typename T, int BM, int BN, int STAGES, int EPI>
__global__ __launch_bounds__(256) void gemm_kernel(GemmArgs<T> a) {
    constexpr int WAVES_M = 2, WAVES_N = 2, NW = 4;
    constexpr int WM = BM / WAVES_M, WN = BN / WAVES_N;
    constexpr int FM = WM / 32, FN = WN / 32;
    constexpr int ROWS = BM + BN;
    constexpr int LPW = ROWS / 8 / NW;  // load instructions per wave per slice
    constexpr int STAGE_BYTES = ROWS * 128;
    constexpr int BK = 128 / sizeof(T);  // elements per slice
    constexpr int KS = BK / 16;          // k16 steps per slice
    static_assert(LPW * 8 * NW == ROWS, "rows per slice must split over the waves");
    static_assert(EPI != EPI_QKVG || WN == 64, "QKVG epilogue needs one head per wave");
    static_assert(EPI != EPI_SWIGLU || FN % 2 == 0, "SWIGLU epilogue needs column pairs");

    extern __shared__ __attribute__((aligned(1024))) unsigned char smem[];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int tiles_m = (a.M + BM - 1) / BM;
    const int pid = xcd_remap(blockIdx.x, gridDim.x);
    const int tile_m = pid % tiles_m, tile_n = pid / tiles_m;
    const int m0 = tile_m * BM, n0 = tile_n * BN;
    const int wm0 = (wave / WAVES_N) * WM, wn0 = (wave % WAVES_N) * WN;
    const int K = a.K;

    // Source of each of this wave's load instructions: stage row r = 8 * (instr) + lane/8,
    // physical chunk lane % 8 <- logical chunk swz(r, lane % 8).  A rows past M are
    // clamped into range (their results are never stored).
    const T* src[LPW];
#pragma unroll
    for (int i = 0; i < LPW; i++) {
        int r = (wave * LPW + i) * 8 + lane / 8;
        int lc = swz(r, lane % 8);
        const T* base;
        if (r < BM) {
            int gr = m0 + r < a.M ? m0 + r : a.M - 1;
            base = a.A + (size_t)gr * K;
        } else {
            base = a.W + (size_t)(n0 + r - BM) * K;
        }
        src[i] = base + lc * (16 / sizeof(T));
    }
#define GEMM_ISSUE(kt_, stage_)                                                            \
    do {                                                                                   \
        unsigned char* dst_ = smem + (stage_) * STAGE_BYTES + wave * LPW * 1024;           \
        _Pragma("unroll") for (int i_ = 0; i_ < LPW; i_++)                                 \
            load_lds16(src[i_] + (size_t)(kt_) * BK, dst_ + i_ * 1024);                    \
    } while (0)

    f32x16 acc[FM][FN];
#pragma unroll
    for (int i = 0; i < FM; i++)
#pragma unroll
        for (int j = 0; j < FN; j++)
#pragma unroll
            for (int e = 0; e < 16; e++) acc[i][j][e] = 0.f;

    const int nk = K / BK;
#pragma unroll
    for (int s = 0; s < STAGES - 1; s++)
        if (s < nk) GEMM_ISSUE(s, s);
    const int fr = lane & 31, fh = lane >> 5;
    for (int kt = 0; kt < nk; kt++) {
        // Slice kt has landed (later slices may still be in flight); make it visible.
        if (STAGES == 3 && kt + 1 < nk) wait_vmcnt<LPW>();
        else if (STAGES == 4 && kt + 2 < nk) wait_vmcnt<2 * LPW>();
        else wait_vmcnt<0>();
        raw_barrier();
        if (kt + STAGES - 1 < nk) GEMM_ISSUE(kt + STAGES - 1, (kt + STAGES - 1) % STAGES);
        const unsigned char* st = smem + (kt % STAGES) * STAGE_BYTES;
#pragma unroll
        for (int ks = 0; ks < KS; ks++) {
            Frag32<T> af[FM], bfr[FN];
#pragma unroll
            for (int i = 0; i < FM; i++) af[i] = read_frag<T>(st, wm0 + 32 * i + fr, ks, fh);
#pragma unroll
            for (int j = 0; j < FN; j++) bfr[j] = read_frag<T>(st, BM + wn0 + 32 * j + fr, ks, fh);
#pragma unroll
            for (int i = 0; i < FM; i++)
#pragma unroll
                for (int j = 0; j < FN; j++) mma32(acc[i][j], af[i], bfr[j]);
        }
    }
#undef GEMM_ISSUE

    // ---- epilogues.  acc[i][j][e] = C[row][col] with
    //      row = m0 + wm0 + 32 i + 8 (e / 4) + 4 (lane / 32) + e % 4,
    //      col = n0 + wn0 + 32 j + lane % 32.
    const int rbase = m0 + wm0 + 4 * (lane >> 5);
    const int cl = lane & 31;
    if constexpr (EPI == EPI_STORE) {
#pragma unroll
        for (int i = 0; i < FM; i++)
#pragma unroll
            for (int e = 0; e < 16; e++) {
                int row = rbase + 32 * i + 8 * (e >> 2) + (e & 3);
                if (row >= a.M) continue;
#pragma unroll
                for (int j = 0; j < FN; j++) a.C[(size_t)row * a.N + n0 + wn0 + 32 * j + cl] = acc[i][j][e];
            }
    } else if constexpr (EPI == EPI_RESID) {
#pragma unroll
        for (int i = 0; i < FM; i++)
#pragma unroll
            for (int e = 0; e < 16; e++) {
                int row = rbase + 32 * i + 8 * (e >> 2) + (e & 3);
                if (row >= a.M) continue;
                const float* g = gate_vec(a.mt, row / a.S, a.layer, a.kind, a.N);
#pragma unroll
                for (int j = 0; j < FN; j++) {
                    int col = n0 + wn0 + 32 * j + cl;
                    float* xp = a.x + (size_t)row * a.N + col;
                    *xp = *xp + g[col] * acc[i][j][e];
                }
            }
    } else if constexpr (EPI == EPI_SWIGLU) {
        // W rows come in 32-row groups alternating W1 / W3 columns: block j even holds
        // u1 and block j+1 the matching u3 for output columns 32 * pair + lane % 32.
        const int half_n = a.N / 2;
#pragma unroll
        for (int i = 0; i < FM; i++)
#pragma unroll
            for (int e = 0; e < 16; e++) {
                int row = rbase + 32 * i + 8 * (e >> 2) + (e & 3);
                if (row >= a.M) continue;
#pragma unroll
                for (int j = 0; j < FN; j += 2) {
                    int pair = (n0 + wn0) / 64 + j / 2;
                    float u1 = acc[i][j][e], u3 = acc[i][j + 1][e];
                    a.U[(size_t)row * half_n + pair * 32 + cl] = from_f32<T>(silu_f(u1) * u3);
                }
            }
    } else if constexpr (EPI == EPI_QKVG) {
        const int D = a.D, Dh = 64;
        const int col0 = n0 + wn0;  // first column of this wave's head
        const int region = col0 / D;
        const int h = (col0 % D) / Dh;
        const int half_heads = a.H / 2;
        if (region <= 1) {
            const float* nw = (region == 0 ? a.q_norm : a.k_norm) + h * Dh;
            T* dst = region == 0 ? a.Q : a.Kd;
#pragma unroll
            for (int i = 0; i < FM; i++)
#pragma unroll
                for (int e = 0; e < 16; e++) {
                    int row = rbase + 32 * i + 8 * (e >> 2) + (e & 3);
                    float ss = acc[i][0][e] * acc[i][0][e] + acc[i][1][e] * acc[i][1][e];
                    ss += __shfl_xor(ss, 1, 64);
                    ss += __shfl_xor(ss, 2, 64);
                    ss += __shfl_xor(ss, 4, 64);
                    ss += __shfl_xor(ss, 8, 64);
                    ss += __shfl_xor(ss, 16, 64);
                    float rms = sqrtf(ss / (float)Dh + a.eps);
                    int rr = row < a.M ? row : a.M - 1;
                    int b = rr / a.S, s = rr % a.S;
#pragma unroll
                    for (int j = 0; j < 2; j++) {
                        int d = 32 * j + cl;
                        float y = acc[i][j][e] / rms * nw[d];
                        float partner = __shfl_xor(y, 1, 64);
                        if (h < half_heads) {
                            int k = d >> 1;
                            float c = a.rope_cos[s * (Dh / 2) + k], sn = a.rope_sin[s * (Dh / 2) + k];
                            y = (d & 1) ? (partner * sn + y * c) : (y * c - partner * sn);
                        }
                        if (region == 0) y *= a.q_scale;
                        if (row < a.M) dst[(((size_t)b * a.H + h) * a.S + s) * Dh + d] = from_f32<T>(y);
                    }
                }
        } else if (region == 2) {
#pragma unroll
            for (int i = 0; i < FM; i++)
#pragma unroll
                for (int e = 0; e < 16; e++) {
                    int row = rbase + 32 * i + 8 * (e >> 2) + (e & 3);
                    if (row >= a.M) continue;
                    int b = row / a.S, s = row % a.S;
                    // V^T in the key order the attention kernel's A operand wants.
                    int pos = sizeof(T) == 2 ? vt_pos_bf16(s) : vt_pos_f32(s);
#pragma unroll
                    for (int j = 0; j < 2; j++) {
                        int d = 32 * j + cl;
                        a.Vd[(((size_t)b * a.H + h) * Dh + d) * a.vt_stride + pos] = from_f32<T>(acc[i][j][e]);
                    }
                }
        } else {
#pragma unroll
            for (int i = 0; i < FM; i++)
#pragma unroll
                for (int e = 0; e < 16; e++) {
                    int row = rbase + 32 * i + 8 * (e >> 2) + (e & 3);
                    if (row >= a.M) continue;
#pragma unroll
                    for (int j = 0; j < 2; j++) {
                        int col = col0 - 3 * D + 32 * j + cl;
                        a.G[(size_t)row * D + col] = from_f32<T>(sigmoid_f(acc[i][j][e]));
                    }
                }
        }
    }
}

template <typename T, int BM, int BN, int STAGES, int EPI>
int launch_cfg(const GemmArgs<T>& a, hipStream_t st) {
    constexpr int BK = 128 / sizeof(T);
    if (a.M <= 0 || a.N % BN != 0 || a.K % BK != 0 || a.K <= 0) return -1;
    int tiles = ((a.M + BM - 1) / BM) * (a.N / BN);
    size_t lds = (size_t)STAGES * (BM + BN) * 128;
    static bool attr_set = false;  // per instantiation; the attribute is process-wide
    if (!attr_set) {
        if (hipFuncSetAttribute((const void*)gemm_kernel<T, BM, BN, STAGES, EPI>,
                                hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds) != hipSuccess)
            return -2;
        attr_set = true;
    }
    gemm_kernel<T, BM, BN, STAGES, EPI><<<tiles, 256, lds, st>>>(a);
    return 0;
}

}  // namespace

// Tile choice per epilogue: the wide projections (QKV+gate, W1|W3) use 128x128 tiles in
// two stages (two workgroups per CU); the D-wide projections (Wo, W2) use 64x64 tiles in
// four stages so that M = 1500 x N = 1024 still yields 384 workgroups for 256 CUs.
template <typename T>
int launch_gemm(int epi, const GemmArgs<T>& a, hipStream_t st) {
    switch (epi) {
        case EPI_STORE: return launch_cfg<T, 64, 64, 4, EPI_STORE>(a, st);
        case EPI_RESID: return launch_cfg<T, 64, 64, 4, EPI_RESID>(a, st);
        case EPI_SWIGLU: return launch_cfg<T, 128, 128, 2, EPI_SWIGLU>(a, st);
        case EPI_QKVG: return launch_cfg<T, 128, 128, 2, EPI_QKVG>(a, st);
    }
    return -1;
}

template int launch_gemm<bf16>(int, const GemmArgs<bf16>&, hipStream_t);
template int launch_gemm<float>(int, const GemmArgs<float>&, hipStream_t);

}  // namespace irodori
