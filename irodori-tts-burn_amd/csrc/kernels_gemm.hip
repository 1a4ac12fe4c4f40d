// Matrix-core GEMM for the DiT projections: C[M,N] = A[M,K] @ W[N,K]^T with fused
// epilogues.  Both operands are K-contiguous in HBM (weights are re-laid out at ingest),
// so every global load is a 16-byte row segment and every LDS fragment read is a single
// 16-byte ds_read.  256 threads = 4 wavefronts in a WAVES_M x WAVES_N grid; K advances
// in 128-byte slices (64 bf16 / 32 f32) through a double-buffered LDS tile with register
// prefetch of the next slice, one barrier per slice.  bf16 uses
// v_mfma_f32_16x16x32_bf16; the f32 path uses v_mfma_f32_16x16x4_f32 on the same
// fragment layout.
//
// Epilogues (all in registers, no extra pass over HBM):
//   EPI_STORE  C f32
//   EPI_RESID  x += gate * C            (gated residual, diffusion.rs:98 / :104)
//   EPI_SWIGLU U = silu(C1) * C3        (feed_forward.rs:80-84; W rows interleaved per 16)
//   EPI_QKVG   q,k: head RMSNorm (norm.rs:60-74) + half RoPE (rope.rs:82-135);
//              v: scatter to [B,H,S,Dh]; gate: sigmoid (attention.rs:423)
#include "common.hpp"
#include "kernels.hpp"

namespace irodori {

namespace {

constexpr int kSliceBytes = 128;
constexpr int kPadBytes = 16;

template <typename T>
__device__ __forceinline__ Frag<T> lds_frag(const T* p);
template <>
__device__ __forceinline__ Frag<bf16> lds_frag<bf16>(const bf16* p) {
    Frag<bf16> f;
    f.v = *reinterpret_cast<const bf16x8*>(p);
    return f;
}
template <>
__device__ __forceinline__ Frag<float> lds_frag<float>(const float* p) {
    Frag<float> f;
    float4 lo = *reinterpret_cast<const float4*>(p);
    float4 hi = *reinterpret_cast<const float4*>(p + 4);
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

template <typename T, int BM, int BN, int WAVES_M, int WAVES_N, int EPI>
__global__ __launch_bounds__(256) void gemm_kernel(GemmArgs<T> a) {
    constexpr int BK = kSliceBytes / sizeof(T);          // elements per K slice
    constexpr int LDSK = BK + kPadBytes / sizeof(T);      // LDS row stride (elements)
    constexpr int VEC = 16 / sizeof(T);                   // elements per 16-byte chunk
    constexpr int WM = BM / WAVES_M, WN = BN / WAVES_N;
    constexpr int FM = WM / 16, FN = WN / 16;
    constexpr int A_LOADS = BM * 8 / 256, B_LOADS = BN * 8 / 256;
    static_assert(WAVES_M * WAVES_N == 4, "4 wavefronts");
    static_assert(A_LOADS >= 1 && B_LOADS >= 1, "tile too small");
    static_assert(EPI != EPI_QKVG || WN == 64, "QKVG epilogue needs one head per wave");
    static_assert(EPI != EPI_SWIGLU || FN % 2 == 0, "SWIGLU epilogue needs column pairs");

    __shared__ __attribute__((aligned(16))) T As[2][BM * LDSK];
    __shared__ __attribute__((aligned(16))) T Bs[2][BN * LDSK];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int tiles_m = (a.M + BM - 1) / BM;
    const int pid = xcd_remap(blockIdx.x, gridDim.x);
    const int tile_m = pid % tiles_m, tile_n = pid / tiles_m;
    const int m0 = tile_m * BM, n0 = tile_n * BN;
    const int wm0 = (wave / WAVES_N) * WM, wn0 = (wave % WAVES_N) * WN;
    const int K = a.K;

    // This thread's 16-byte chunks of the A and W slices: chunk c = tid + 256 i covers row
    // c / 8, elements (c % 8) * VEC.. of the slice.  A rows past M are clamped into range
    // (their results are never stored).
    const int crow = tid >> 3, ccol = (tid & 7) * VEC;
    const T* ga0 = a.A + ccol;
    const T* gb0 = a.W + (size_t)n0 * K + ccol;
    int arow[A_LOADS];
#pragma unroll
    for (int i = 0; i < A_LOADS; i++) {
        int r = m0 + crow + 32 * i;
        arow[i] = r < a.M ? r : a.M - 1;
    }
    u32x4 ra[A_LOADS], rb[B_LOADS];
#define GEMM_GLOAD(k0)                                                                     \
    do {                                                                                   \
        _Pragma("unroll") for (int i = 0; i < A_LOADS; i++) ra[i] =                        \
            *reinterpret_cast<const u32x4*>(ga0 + (size_t)arow[i] * K + (k0));             \
        _Pragma("unroll") for (int i = 0; i < B_LOADS; i++) rb[i] =                        \
            *reinterpret_cast<const u32x4*>(gb0 + (size_t)(crow + 32 * i) * K + (k0));     \
    } while (0)
#define GEMM_LSTORE(buf)                                                                   \
    do {                                                                                   \
        _Pragma("unroll") for (int i = 0; i < A_LOADS; i++)                                \
            *reinterpret_cast<u32x4*>(&As[buf][(crow + 32 * i) * LDSK + ccol]) = ra[i];    \
        _Pragma("unroll") for (int i = 0; i < B_LOADS; i++)                                \
            *reinterpret_cast<u32x4*>(&Bs[buf][(crow + 32 * i) * LDSK + ccol]) = rb[i];    \
    } while (0)

    f32x4 acc[FM][FN];
#pragma unroll
    for (int i = 0; i < FM; i++)
#pragma unroll
        for (int j = 0; j < FN; j++) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

    const int nk = K / BK;
    GEMM_GLOAD(0);
    GEMM_LSTORE(0);
    __syncthreads();
    const int fr = lane & 15, fk = (lane >> 4) * 8;
    for (int kt = 0; kt < nk; kt++) {
        const int buf = kt & 1;
        if (kt + 1 < nk) GEMM_GLOAD((kt + 1) * BK);
        const T* as = As[buf];
        const T* bs = Bs[buf];
#pragma unroll
        for (int kc = 0; kc < BK / 32; kc++) {
            Frag<T> af[FM], bfr[FN];
#pragma unroll
            for (int i = 0; i < FM; i++) af[i] = lds_frag<T>(as + (wm0 + 16 * i + fr) * LDSK + kc * 32 + fk);
#pragma unroll
            for (int j = 0; j < FN; j++) bfr[j] = lds_frag<T>(bs + (wn0 + 16 * j + fr) * LDSK + kc * 32 + fk);
#pragma unroll
            for (int i = 0; i < FM; i++)
#pragma unroll
                for (int j = 0; j < FN; j++) mma16(acc[i][j], af[i], bfr[j]);
        }
        if (kt + 1 < nk) GEMM_LSTORE(buf ^ 1);
        __syncthreads();
    }

#undef GEMM_GLOAD
#undef GEMM_LSTORE

    // ---- epilogues. acc[i][j][e] = C[m0+wm0+16i+4*(lane/16)+e][n0+wn0+16j+lane%16] ----
    const int rbase = m0 + wm0 + 4 * (lane >> 4);
    const int cbase = n0 + wn0 + (lane & 15);
    if constexpr (EPI == EPI_STORE) {
#pragma unroll
        for (int i = 0; i < FM; i++)
#pragma unroll
            for (int e = 0; e < 4; e++) {
                int row = rbase + 16 * i + e;
                if (row >= a.M) continue;
#pragma unroll
                for (int j = 0; j < FN; j++) a.C[(size_t)row * a.N + cbase + 16 * j] = acc[i][j][e];
            }
    } else if constexpr (EPI == EPI_RESID) {
#pragma unroll
        for (int i = 0; i < FM; i++)
#pragma unroll
            for (int e = 0; e < 4; e++) {
                int row = rbase + 16 * i + e;
                if (row >= a.M) continue;
                const float* g = gate_vec(a.mt, row / a.S, a.layer, a.kind, a.N);
#pragma unroll
                for (int j = 0; j < FN; j++) {
                    int col = cbase + 16 * j;
                    float* xp = a.x + (size_t)row * a.N + col;
                    *xp = *xp + g[col] * acc[i][j][e];
                }
            }
    } else if constexpr (EPI == EPI_SWIGLU) {
        const int half_n = a.N / 2;
#pragma unroll
        for (int i = 0; i < FM; i++)
#pragma unroll
            for (int e = 0; e < 4; e++) {
                int row = rbase + 16 * i + e;
                if (row >= a.M) continue;
#pragma unroll
                for (int j = 0; j < FN; j += 2) {
                    int pair = (n0 + wn0) / 32 + j / 2;
                    float u1 = acc[i][j][e], u3 = acc[i][j + 1][e];
                    a.U[(size_t)row * half_n + pair * 16 + (lane & 15)] = from_f32<T>(silu_f(u1) * u3);
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
                for (int e = 0; e < 4; e++) {
                    int row = rbase + 16 * i + e;
                    float ss = 0.f;
#pragma unroll
                    for (int j = 0; j < FN; j++) ss += acc[i][j][e] * acc[i][j][e];
                    ss += __shfl_xor(ss, 1, 64);
                    ss += __shfl_xor(ss, 2, 64);
                    ss += __shfl_xor(ss, 4, 64);
                    ss += __shfl_xor(ss, 8, 64);
                    float rms = sqrtf(ss / (float)Dh + a.eps);
                    int rr = row < a.M ? row : a.M - 1;
                    int b = rr / a.S, s = rr % a.S;
#pragma unroll
                    for (int j = 0; j < FN; j++) {
                        int d = 16 * j + (lane & 15);
                        float y = acc[i][j][e] / rms * nw[d];
                        float partner = __shfl_xor(y, 1, 64);
                        if (h < half_heads) {
                            int k = d >> 1;
                            float c = a.rope_cos[s * (Dh / 2) + k], sn = a.rope_sin[s * (Dh / 2) + k];
                            y = (d & 1) ? (partner * sn + y * c) : (y * c - partner * sn);
                        }
                        if (row < a.M)
                            dst[(((size_t)b * a.H + h) * a.S + s) * Dh + d] = from_f32<T>(y);
                    }
                }
        } else if (region == 2) {
#pragma unroll
            for (int i = 0; i < FM; i++)
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    int row = rbase + 16 * i + e;
                    if (row >= a.M) continue;
                    int b = row / a.S, s = row % a.S;
#pragma unroll
                    for (int j = 0; j < FN; j++) {
                        int d = 16 * j + (lane & 15);
                        a.Vd[(((size_t)b * a.H + h) * a.S + s) * Dh + d] = from_f32<T>(acc[i][j][e]);
                    }
                }
        } else {
#pragma unroll
            for (int i = 0; i < FM; i++)
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    int row = rbase + 16 * i + e;
                    if (row >= a.M) continue;
#pragma unroll
                    for (int j = 0; j < FN; j++) {
                        int col = col0 - 3 * D + 16 * j + (lane & 15);
                        a.G[(size_t)row * D + col] = from_f32<T>(sigmoid_f(acc[i][j][e]));
                    }
                }
        }
    }
}

template <typename T, int BM, int BN, int WAVES_M, int WAVES_N, int EPI>
int launch_cfg(const GemmArgs<T>& a, hipStream_t st) {
    constexpr int BK = kSliceBytes / sizeof(T);
    if (a.M <= 0 || a.N % BN != 0 || a.K % BK != 0 || a.K <= 0) return -1;
    int tiles = ((a.M + BM - 1) / BM) * (a.N / BN);
    gemm_kernel<T, BM, BN, WAVES_M, WAVES_N, EPI><<<tiles, 256, 0, st>>>(a);
    return 0;
}

}  // namespace

// Tile choice per epilogue: the wide projections (QKV+gate, W1|W3) use 128x128 tiles
// with one 64x64 block per wavefront; the D-wide projections (Wo, W2) use 64x64 tiles
// so that M = 1500 x N = 1024 still yields 384 workgroups for 256 CUs.
template <typename T>
int launch_gemm(int epi, const GemmArgs<T>& a, hipStream_t st) {
    switch (epi) {
        case EPI_STORE: return launch_cfg<T, 64, 64, 2, 2, EPI_STORE>(a, st);
        case EPI_RESID: return launch_cfg<T, 64, 64, 2, 2, EPI_RESID>(a, st);
        case EPI_SWIGLU: return launch_cfg<T, 128, 128, 2, 2, EPI_SWIGLU>(a, st);
        case EPI_QKVG: return launch_cfg<T, 128, 128, 2, 2, EPI_QKVG>(a, st);
    }
    return -1;
}

template int launch_gemm<bf16>(int, const GemmArgs<bf16>&, hipStream_t);
template int launch_gemm<float>(int, const GemmArgs<float>&, hipStream_t);

}  // namespace irodori
