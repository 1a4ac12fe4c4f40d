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
//   EPI_ADD    x = (x + C) * rmask[row]  (encoder residual + re-mask)
//   EPI_SNAKE  U = Snake(C + bias)       (codec ResidualUnit's dilated conv + act1)
//   EPI_RESUNIT x += Snake(C + bias) @ W2^T + bias2 (the whole ResidualUnit tail: the
//              Snake'd tile goes through LDS into a second MFMA pass over the 1x1 conv)
// The STORE / ADD epilogues add an optional bias[col].  With CONV set (launch_gemm_conv)
// the A tile of slice kt is the implicit im2col of a convolution: the slice lies in one
// tap j = kt * BK / conv_cp, whose source rows sit j * conv_dil rows further down, so only
// the buffer offset of the A loads changes; the LDS layout and the MFMA loop are the same.
//   EPI_QKVG   q,k: head RMSNorm (norm.rs:60-74) + half RoPE (rope.rs:82-135);
//              q pre-scaled by Dh^-1/2 log2(e) for the attention softmax;
//              v: scatter to V^T [B,H,Dh,S'] (key-permuted); gate: sigmoid (attention.rs:423)
#include <type_traits>

#include "common.hpp"
#include "kernels.hpp"

namespace irodori {

namespace {

typedef float f32x16 __attribute__((ext_vector_type(16)));

template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}
// Wait until at most `ahead` (<= MAXA) slices of LPW loads each are still in flight.
template <int MAXA, int LPW>
__device__ __forceinline__ void wait_slices(int ahead) {
    if constexpr (MAXA <= 0) {
        wait_vmcnt<0>();
    } else {
        static_assert(MAXA * LPW <= 63, "vmcnt holds 6 bits");
        if (ahead >= MAXA) wait_vmcnt<MAXA * LPW>();
        else wait_slices<MAXA - 1, LPW>(ahead);
    }
}
// Workgroup barrier without the implied memory fence (which would drain every in-flight
// load, including the prefetched slices).
__device__ __forceinline__ void raw_barrier() { asm volatile("s_barrier" ::: "memory"); }

// 16 bytes per lane from a raw buffer straight into LDS (lane i lands at lds + 16 i).
// Offsets at or past the resource's byte count read as zero.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, unsigned bytes) {
    // Raw (stride 0) buffer; dword3 0x00020000 is the gfx9-family data format for raw access.
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}
__device__ __forceinline__ void buf_load_lds16(__amdgpu_buffer_rsrc_t r, unsigned voff, unsigned soff, void* lds) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)lds, 16, voff, soff, 0, 0);
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

// fp8 fragment of one 32x32x64 step: 32 bytes per lane, k = 16*(lane/32) + 0..15 (the
// first 32-wide scale block) and 32 + 16*(lane/32) + 0..15 (the second), i.e. 16-byte
// chunks 4*ks + h and 4*ks + 2 + h of the 128-byte row.  The E8M0 scale of row r, block b
// is supplied by lane r + 32 b.
typedef int i32x8 __attribute__((ext_vector_type(8)));
struct Frag8 {
    i32x8 v;
};
__device__ __forceinline__ Frag8 read_frag8(const unsigned char* st, int r, int ks, int h) {
    const int4 lo = *reinterpret_cast<const int4*>(st + r * 128 + (swz(r, 4 * ks + h) << 4));
    const int4 hi = *reinterpret_cast<const int4*>(st + r * 128 + (swz(r, 4 * ks + 2 + h) << 4));
    Frag8 f;
    f.v[0] = lo.x; f.v[1] = lo.y; f.v[2] = lo.z; f.v[3] = lo.w;
    f.v[4] = hi.x; f.v[5] = hi.y; f.v[6] = hi.z; f.v[7] = hi.w;
    return f;
}
__device__ __forceinline__ void mma8(f32x16& acc, const Frag8& a, const Frag8& b, int scale_a) {
    // cbsz = blgp = 0: both operands e4m3; B's block scale is 2^0 (E8M0 127).
    acc = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a.v, b.v, acc, 0, 0, 0, scale_a, 0, 127);
}

// Sum over the 32 lanes of each half-wave (lanes 0-31 and 32-63 separately): DPP
// rotations within 16-lane rows, then v_permlane16_swap, which exchanges the odd 16-lane
// rows of one operand with the even rows of the other.  With both operands equal to v the
// two results hold, at every lane, the values of lane l and lane l ^ 16, so their sum is
// the half-wave total (all on the VALU; no LDS-pipeline swizzle).
#define IRO_DPP(v, ctrl)                                                                        \
    __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, (v)), (ctrl), 0xF, 0xF, false))
__device__ __forceinline__ float half_wave_sum(float v) {
    v += IRO_DPP(v, 0x128);  // row_ror:8
    v += IRO_DPP(v, 0x124);  // row_ror:4
    v += IRO_DPP(v, 0x4E);   // quad_perm [2,3,0,1]
    v += IRO_DPP(v, 0xB1);   // quad_perm [1,0,3,2]
    const unsigned u = __builtin_bit_cast(unsigned, v);
    const auto sw = __builtin_amdgcn_permlane16_swap(u, u, false, false);
    return __builtin_bit_cast(float, (unsigned)sw[0]) + __builtin_bit_cast(float, (unsigned)sw[1]);
}

// Sums of 16 values per lane over the 32 lanes of each half-wave, one value per row: a
// halving butterfly over lane bits 4, 3, 2, 1 (at each step a lane keeps the lower or upper
// half of its values, by its lane bit, and adds the partner's copy of those), then bit 0.
// v[0] ends as the sum of value e over the half-wave at every lane l with
// e = 8 b4 + 4 b3 + 2 b2 + b1 (the bits of l % 32); returns e.  The order of additions is
// fixed, so the sums are deterministic.
__device__ __forceinline__ int half_wave_row_sums(float (&v)[16], int l) {
#pragma unroll
    for (int n = 16, m = 16; n > 1; n >>= 1, m >>= 1) {
        const bool hi = (l & m) != 0;
#pragma unroll
        for (int k = 0; k < n / 2; k++) {
            // Both values in registers before the selects (else the select of two array
            // elements is folded into a lane-variable register index: a 16-way select chain).
            float lo = v[k], up = v[k + n / 2];
            asm volatile("" : "+v"(lo), "+v"(up));
            const float send = hi ? lo : up;
            const float keep = hi ? up : lo;
            v[k] = keep + __shfl_xor(send, m, 64);
        }
    }
    v[0] += __shfl_xor(v[0], 1, 64);
    return 8 * ((l >> 4) & 1) + 4 * ((l >> 3) & 1) + 2 * ((l >> 2) & 1) + ((l >> 1) & 1);
}

// Staged bf16 wave tile of the QKVG epilogue: row r (< 64) of 64 columns lives at
// slot + 256 r, its 16-byte chunk c at chunk position c ^ (4 * ((r >> 2 ^ r) & 1)).  The
// column writes of an accumulator step touch rows r and r + 4 together and the 16-byte row
// reads rows r and r + 1 together; the xor puts each pair on different banks.
__device__ __forceinline__ int stage_off(int r, int col) {
    const int c = col >> 3;
    return r * 256 + ((c ^ (4 * (((r >> 2) ^ r) & 1))) << 4) + (col & 7) * 2;
}
// The same tile packed at 128 bytes per row (the q / k staging, which shares no row with
// a table): the same chunk xor keeps rows r and r + 4 of a column write on different banks.
__device__ __forceinline__ int stage_off_packed(int r, int col) {
    const int c = col >> 3;
    return r * 128 + ((c ^ (4 * (((r >> 2) ^ r) & 1))) << 4) + (col & 7) * 2;
}

__device__ __forceinline__ const float* gate_vec(const ModTable& mt, int b, int layer, int kind,
                                                int D) {
    int vec = mod_vec_index(mt, mt.step ? *mt.step : 0, b);
    return mt.tab + ((size_t)vec * mt.layers * 6 + (size_t)layer * 6 + kind * 3 + 2) * D;
}

// Four-wave workgroups are sized for two per CU (LDS), so they ask the compiler for two
// waves per SIMD: at most 256 registers per wave, accumulators included.
template <typename T, int BM, int BN, int WAVES_M, int WAVES_N, int STAGES, int EPI, bool F8 = false,
          bool CONV = false>
__global__ __launch_bounds__(64 * WAVES_M * WAVES_N)
__attribute__((amdgpu_waves_per_eu(WAVES_M * WAVES_N == 4 ? 2 : 1))) void gemm_kernel(GemmArgs<T> a) {
    constexpr int NW = WAVES_M * WAVES_N;
    constexpr int WM = BM / WAVES_M, WN = BN / WAVES_N;
    constexpr int FM = WM / 32, FN = WN / 32;
    constexpr int ROWS = BM + BN;
    constexpr int LPW = ROWS / 8 / NW;  // load instructions per wave per slice
    constexpr int STAGE_BYTES = ROWS * 128;
    constexpr int ES = F8 ? 1 : (int)sizeof(T);  // operand element bytes
    constexpr int BK = 128 / ES;                  // elements per slice
    constexpr int KS = BK / (F8 ? 64 : 16);       // MFMA k-steps per slice
    static_assert(!F8 || sizeof(T) == 2, "fp8 operands produce bf16 / f32 outputs");
    static_assert(LPW * 8 * NW == ROWS, "rows per slice must split over the waves");
    static_assert(FM * 32 == WM && FN * 32 == WN, "wave tiles are whole 32x32 blocks");
    static_assert(BM % 8 == 0, "a load instruction covers A rows or W rows, not both");
    static_assert((EPI != EPI_QKVG && EPI != EPI_CTXKV) || WN == 64 || WN == 128,
                  "QKVG / CTXKV epilogues need one 64- or 128-column head per wave");
    static_assert(EPI != EPI_SWIGLU || FN % 2 == 0, "SWIGLU epilogue needs column pairs");
    static_assert(!(F8 && CONV), "convolutions take bf16 / f32 operands");

    extern __shared__ __attribute__((aligned(1024))) unsigned char smem[];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    // Tiles in groups of GM row tiles: consecutive ids (one XCD's, see xcd_remap) sweep
    // the group's GM row tiles for one column tile, then the next column tile, so the
    // workgroups an XCD runs together share GM A tiles and a few W tiles in its L2.  With
    // at most GM row tiles this is the plain column-by-column order.  Measured on the RF
    // run (config 4, 750-row launches), one GM for every GEMM: GM = 1 / 2 / 3 / 4 / 6 / 8 /
    // 16 gave 47.4 / 46.0 / 46.0 / 45.85 / 46.2 / 46.4 / 46.8 ms.  The 64-row W_o / W2 tiles
    // (12 row tiles) decide it; the 128-row tiles run the same at 3, 4 or 8 and keep 8, where
    // every row tile of a weight column shares the column on one XCD (W13 fetches 30 MB per
    // launch instead of 37 at GM = 4).  The codec's convolutions keep 8 (4 was 0.4 % slower
    // there).  The raster never changes a tile's arithmetic.
    constexpr int GM = (CONV || BM >= 128) ? 8 : 4;
    const int tiles_m = (a.M + BM - 1) / BM, tiles_n = a.N / BN;
    const int pid = xcd_remap(blockIdx.x, gridDim.x);
    const int per_group = GM * tiles_n, group = pid / per_group, first_m = group * GM;
    const int gm = tiles_m - first_m < GM ? tiles_m - first_m : GM;
    const int local = pid - group * per_group;
    const int tile_m = first_m + local % gm, tile_n = local / gm;
    const int m0 = tile_m * BM, n0 = tile_n * BN;
    const int wm0 = (wave / WAVES_N) * WM, wn0 = (wave % WAVES_N) * WN;
    const int K = a.K;

    // Load instruction i of this wave fills stage rows 8 (wave*LPW + i) .. +7: lane -> row
    // r = 8 (wave*LPW + i) + lane / 8, physical chunk lane % 8 <- logical chunk
    // swz(r, lane % 8).  One SGPR resource per operand tile; A rows past M fall outside
    // the A resource and read as zero.  The slice offset kt * 128 bytes rides in soffset.
    // CONV: A rows are conv_cp elements apart and the resource spans every source row from
    // m0 on (the taps reach past the tile); rows past conv_rows read as zero.
    const int lda = CONV ? a.conv_cp : K;
    int arows = a.M - m0 < BM ? a.M - m0 : BM;
    if constexpr (CONV) arows = a.conv_rows - m0 > 0 ? a.conv_rows - m0 : 0;
    const unsigned char* Ab = F8 ? a.A8 : reinterpret_cast<const unsigned char*>(a.A);
    const unsigned char* Wb = F8 ? a.W8 : reinterpret_cast<const unsigned char*>(a.W);
    const __amdgpu_buffer_rsrc_t rA = make_rsrc(Ab + (size_t)m0 * lda * ES, (unsigned)((size_t)arows * lda * ES));
    const __amdgpu_buffer_rsrc_t rW = make_rsrc(Wb + (size_t)n0 * K * ES, (unsigned)(BN * K * ES));
    // W row rr of the tile: group rr / 64 at 64 K ES bytes in either layout; within the
    // group rows are K ES bytes apart (row-major) or 128 (tile-major, where consecutive
    // slices are 8 KB apart instead of 128 bytes).
    const bool wt = !CONV && a.w_tiled;
    const unsigned w_row = wt ? 128u : (unsigned)(K * ES), w_slice = wt ? 8192u : 128u;
    unsigned voff[LPW];
#pragma unroll
    for (int i = 0; i < LPW; i++) {
        const int r = (wave * LPW + i) * 8 + lane / 8;
        const int rr = r < BM ? r : r - BM;
        voff[i] = (r < BM ? (unsigned)rr * (unsigned)(lda * ES)
                          : (unsigned)(rr / 64) * (unsigned)(64 * K * ES) + (unsigned)(rr % 64) * w_row) +
                  (unsigned)swz(r, lane % 8) * 16u;
    }
    // CONV: byte offset of slice kt in the A source = kt * 128 (the taps laid end to end),
    // plus (conv_dil - 1) rows for each tap before the slice's tap j0 = kt BK / conv_cp.
    // With conv_cp an odd multiple of BK / 2 a slice can straddle two taps, always at its
    // middle: the lanes loading logical chunks 4..7 then belong to tap j0 + 1 and add one
    // more step (voff_hi).
    [[maybe_unused]] const unsigned conv_dstep = CONV ? (unsigned)((a.conv_dil - 1) * a.conv_cp * ES) : 0u;
    [[maybe_unused]] unsigned voff_hi[LPW];
    if constexpr (CONV) {
#pragma unroll
        for (int i = 0; i < LPW; i++)
            voff_hi[i] = voff[i] + (swz((wave * LPW + i) * 8 + lane / 8, lane % 8) >= 4 ? conv_dstep : 0u);
    }
    // fp8: the tile's E8M0 block scales (BM rows x K/32 bytes) are staged in LDS past the
    // operand stages before the main loop, slice-major: the word of row r for slice kt (its
    // four k blocks) at (kt * BM + r) * 4, so a wave's 32 rows read 32 consecutive words.
    // Rows past M read as 127 (2^0) over zero codes.
    [[maybe_unused]] const int kb = K / 32;
    [[maybe_unused]] unsigned char* sc_lds = smem + STAGES * STAGE_BYTES;
    if constexpr (F8) {
        const int words = BM * (kb / 4);
        for (int idx = threadIdx.x; idx < words; idx += 64 * NW) {
            const int r = idx % BM, c4 = idx / BM;
            unsigned w = 0x7f7f7f7fu;
            if (m0 + r < a.M) w = *reinterpret_cast<const unsigned*>(a.As + (size_t)(m0 + r) * kb + 4 * c4);
            *reinterpret_cast<unsigned*>(sc_lds + (c4 * BM + r) * 4) = w;
        }
        __syncthreads();
    }
#define GEMM_ISSUE(kt_, stage_)                                                            \
    do {                                                                                   \
        unsigned char* dst_ = smem + (stage_) * STAGE_BYTES + wave * LPW * 1024;           \
        const unsigned ws_ = (unsigned)(kt_) * w_slice;                                    \
        unsigned as_ = (unsigned)(kt_) * 128u;                                             \
        bool split_ = false;                                                               \
        if constexpr (CONV) {                                                              \
            const int k0_ = (kt_) * BK, j0_ = k0_ / a.conv_cp;                             \
            as_ += (unsigned)j0_ * conv_dstep;                                             \
            split_ = k0_ - j0_ * a.conv_cp + BK > a.conv_cp;                               \
        }                                                                                  \
        _Pragma("unroll") for (int i_ = 0; i_ < LPW; i_++) {                               \
            const bool isA = (wave * LPW + i_) * 8 < BM;                                   \
            const unsigned vo_ = (CONV && isA && split_) ? voff_hi[i_] : voff[i_];         \
            buf_load_lds16(isA ? rA : rW, vo_, isA ? as_ : ws_, dst_ + i_ * 1024);         \
        }                                                                                  \
    } while (0)

    f32x16 acc[FM][FN];
#pragma unroll
    for (int i = 0; i < FM; i++)
#pragma unroll
        for (int j = 0; j < FN; j++)
#pragma unroll
            for (int e = 0; e < 16; e++) acc[i][j][e] = 0.f;

    // Accumulator element (i, j, e) of this lane is C[row][col] with
    //   row = rbase + 32 i + 8 (e / 4) + e % 4,  col = n0 + wn0 + 32 j + cl.
    const int rbase = m0 + wm0 + 4 * (lane >> 5);
    const int cl = lane & 31;
    const float inv_s = 1.f / (float)a.S;

    // EPI_RESID (S >= 32): the residual elements this lane updates and the gate rows of
    // the (at most two) batch rows each 32-row block touches are loaded before the main
    // loop, so their latency hides behind it (each element belongs to one lane only).
    // With Hn set (fused adaLN producer) the next norm's scale columns are loaded likewise.
    [[maybe_unused]] float xpre[FM][16][FN];
    [[maybe_unused]] float gpre[FM][2][FN];
    [[maybe_unused]] float spre[FM][2][FN];
    [[maybe_unused]] int hi_row[FM];  // first row of the upper batch row of block i
    if constexpr (EPI == EPI_RESID) {
        if (a.S >= 32) {
            const int step = a.mt.step ? *a.mt.step : 0;
#pragma unroll
            for (int i = 0; i < FM; i++) {
                const int r0 = rbase + 32 * i;
                int b_lo, s_lo;
                row_bs(r0 < a.M ? r0 : a.M - 1, a.S, inv_s, b_lo, s_lo);
                const int b_hi = b_lo + 1;
                hi_row[i] = b_hi * a.S;
                const bool need_hi = s_lo + 28 >= a.S && hi_row[i] < a.M;  // block may cross into b_hi
#pragma unroll
                for (int u = 0; u < 2; u++) {
                    const int bb = u ? b_hi : b_lo;
                    const float* g = a.mt.tab + ((size_t)mod_vec_index(a.mt, step, bb) * a.mt.layers * 6 +
                                                 (size_t)a.layer * 6 + a.kind * 3 + 2) * a.N;
#pragma unroll
                    for (int j = 0; j < FN; j++) gpre[i][u][j] = (!u || need_hi) ? g[n0 + wn0 + 32 * j + cl] : 0.f;
                    if (!F8 && a.Hn) {
                        const float* sc = a.mt.tab + ((size_t)mod_vec_index(a.mt, step, bb) * a.mt.layers * 6 +
                                                      (size_t)a.next_layer * 6 + a.next_kind * 3 + 1) * a.N;
#pragma unroll
                        for (int j = 0; j < FN; j++) spre[i][u][j] = (!u || need_hi) ? sc[n0 + wn0 + 32 * j + cl] : 0.f;
                    }
                }
#pragma unroll
                for (int e = 0; e < 16; e++) {
                    const int row = r0 + 8 * (e >> 2) + (e & 3);
#pragma unroll
                    for (int j = 0; j < FN; j++)
                        xpre[i][e][j] = row < a.M ? a.x[(size_t)row * a.N + n0 + wn0 + 32 * j + cl] : 0.f;
                }
            }
        }
    }

    // Fused adaLN consumer: lane l of a wave loads the K/32 partial sums of rows m0 + wm0 + l
    // (+ 64) and this wave's shift-bias columns before the operand stream starts, so their
    // latency hides behind it; iteration 0 of the main loop turns the sums into r = rsqrt(mean
    // x^2 + eps), kept in registers until the stage buffers are free after the main loop.
    constexpr bool FUSE_IN = !F8 && (EPI == EPI_QKVG || EPI == EPI_SWIGLU);
    constexpr int RPL = (WM + 63) / 64;  // rows of the wave per lane
    [[maybe_unused]] float4 rsv[RPL][16];
    [[maybe_unused]] float rown[RPL];
    [[maybe_unused]] float bc[FN];
    if constexpr (FUSE_IN) {
        static_assert(RPL <= 3, "at most three rows per lane");
        static_assert(STAGES * STAGE_BYTES >= NW * WM * 4, "row scales are staged in the operand buffers");
        if (a.rstat) {
            const int vec = mod_vec_index(a.mt, a.mt.step ? *a.mt.step : 0, 0);
#pragma unroll
            for (int j = 0; j < FN; j++) bc[j] = a.rbias[(size_t)vec * a.N + n0 + wn0 + 32 * j + lane % 32];
            const int nq = K / 128;
#pragma unroll
            for (int p = 0; p < RPL; p++) {
                const int rl = 64 * p + lane, row = m0 + wm0 + rl;
#pragma unroll
                for (int q = 0; q < 16; q++) rsv[p][q] = make_float4(0.f, 0.f, 0.f, 0.f);
                if (rl < WM && row < a.M) {
                    const float4* pp = reinterpret_cast<const float4*>(a.rstat + (size_t)row * (K / 32));
#pragma unroll
                    for (int q = 0; q < 16; q++)
                        if (q < nq) rsv[p][q] = pp[q];
                }
            }
        }
    }

    const int nk = K / BK;
    // QKVG tiles holding a RoPE head (q or k, head < H / 2): the table rows of the tile's BM
    // tokens, (cos, sin) pairs [S, 32, 2] f32 = 256 bytes per token, go into LDS by the same
    // buffer-to-LDS loads as the operands, 1 KB (4 tokens) per instruction; token
    // m0 + 4 j + lane / 16 lands at 256 (4 j) + 16 lane.  With S >= 4 the token index steps
    // by 4 with one wrap at most (rows past M read a valid table row, unused).
    // The tile needs them when any of its 64-column heads does: with D an odd multiple of 64
    // a tile can start on the last q head (no RoPE) and end on k head 0 (RoPE).
    // (128-dim heads read their table rows from global memory in the epilogue.)
    [[maybe_unused]] bool rope_wg = false;
    if constexpr (EPI == EPI_QKVG && WN == 64) {
#pragma unroll
        for (int c = n0; c < n0 + BN; c += 64) rope_wg = rope_wg || (c / a.D <= 1 && (c % a.D) / 64 < a.H / 2);
    }
    [[maybe_unused]] auto rope_rows_issue = [&](unsigned char* dst) {
        static_assert(EPI != EPI_QKVG || (BM * 256 <= STAGE_BYTES && (BM * 256 / 1024) % NW == 0),
                      "RoPE rows fill whole stage instructions");
        constexpr int RI = BM * 256 / 1024 / NW;  // instructions per wave
        const __amdgpu_buffer_rsrc_t rT = make_rsrc(a.rope_cs, (unsigned)a.S * 256u);
        const int r0 = m0 + 4 * wave * RI + lane / 16;
        int bq, sq;
        row_bs(min(r0, a.M - 1), a.S, inv_s, bq, sq);
#pragma unroll
        for (int j = 0; j < RI; j++) {
            if (a.S < 4) row_bs(min(r0 + 4 * j, a.M - 1), a.S, inv_s, bq, sq);
            buf_load_lds16(rT, (unsigned)sq * 256u + (unsigned)(lane % 16) * 16u, 0u, dst + (wave * RI + j) * 1024);
            sq += 4;
            sq = sq >= a.S ? sq - a.S : sq;
        }
    };
#pragma unroll
    for (int s = 0; s < STAGES - 1; s++)
        if (s < nk) GEMM_ISSUE(s, s);
    const int fr = lane & 31, fh = lane >> 5;
    for (int kt = 0; kt < nk; kt++) {
        // Slice kt has landed (the min(STAGES - 2, nk - 1 - kt) slices issued after it may
        // still be in flight); make it visible.
        wait_slices<STAGES - 2, LPW>(nk - 1 - kt);
        raw_barrier();
        if (kt + STAGES - 1 < nk) GEMM_ISSUE(kt + STAGES - 1, (kt + STAGES - 1) % STAGES);
        if constexpr (EPI == EPI_QKVG) {
            // The stage after the last slice's was last read in iteration nk - 2, which every
            // wave has finished at this barrier: the RoPE rows of the tile stream into it
            // while the last slice's MFMAs run.
            if (rope_wg && kt == nk - 1) rope_rows_issue(smem + (nk % STAGES) * STAGE_BYTES);
        }
        if constexpr (FUSE_IN) {
            if (a.rstat && kt == 0) {
#pragma unroll
                for (int p = 0; p < RPL; p++) {
                    float ss = 0.f;
#pragma unroll
                    for (int q = 0; q < 16; q++) {
                        ss += rsv[p][q].x;
                        ss += rsv[p][q].y;
                        ss += rsv[p][q].z;
                        ss += rsv[p][q].w;
                    }
                    rown[p] = m0 + wm0 + 64 * p + lane < a.M ? 1.f / sqrtf(ss / (float)K + a.eps) : 1.f;
                }
            }
        }
        const unsigned char* st = smem + (kt % STAGES) * STAGE_BYTES;
        if constexpr (F8) {
            // Scale bytes of this lane's rows for the slice's four k blocks.
            unsigned scw[FM];
#pragma unroll
            for (int i = 0; i < FM; i++) scw[i] = *reinterpret_cast<const unsigned*>(sc_lds + (kt * BM + wm0 + 32 * i + fr) * 4);
            // Fragments double-buffered as in the bf16 loop: the reads of step ks + 1 go out
            // ahead of the MFMAs of step ks (two 16-byte LDS reads per fragment).
            Frag8 af8[2][FM], bf8[2][FN];
#pragma unroll
            for (int i = 0; i < FM; i++) af8[0][i] = read_frag8(st, wm0 + 32 * i + fr, 0, fh);
#pragma unroll
            for (int j = 0; j < FN; j++) bf8[0][j] = read_frag8(st, BM + wn0 + 32 * j + fr, 0, fh);
            __builtin_amdgcn_sched_group_barrier(0x100, 2 * (FM + FN), 0);
#pragma unroll
            for (int ks = 0; ks < KS; ks++) {
                const int cur = ks & 1, nxt = cur ^ 1;
                if (ks + 1 < KS) {
#pragma unroll
                    for (int i = 0; i < FM; i++) af8[nxt][i] = read_frag8(st, wm0 + 32 * i + fr, ks + 1, fh);
#pragma unroll
                    for (int j = 0; j < FN; j++) bf8[nxt][j] = read_frag8(st, BM + wn0 + 32 * j + fr, ks + 1, fh);
                }
#pragma unroll
                for (int i = 0; i < FM; i++) {
                    const int sa = (int)((scw[i] >> (8 * (2 * ks + fh))) & 0xffu);
#pragma unroll
                    for (int j = 0; j < FN; j++) mma8(acc[i][j], af8[cur][i], bf8[cur][j], sa);
                }
                if (ks + 1 < KS) __builtin_amdgcn_sched_group_barrier(0x100, 2 * (FM + FN), 0);  // DS reads
                __builtin_amdgcn_sched_group_barrier(0x008, FM * FN, 0);                         // MFMAs
            }
            continue;
        }
        // Fragments double-buffered in registers: the LDS reads of k16 step ks + 1 are
        // issued ahead of the MFMAs of step ks, so their latency hides behind FM*FN MFMAs.
        Frag32<T> af[2][FM], bfr[2][FN];
#pragma unroll
        for (int i = 0; i < FM; i++) af[0][i] = read_frag<T>(st, wm0 + 32 * i + fr, 0, fh);
#pragma unroll
        for (int j = 0; j < FN; j++) bfr[0][j] = read_frag<T>(st, BM + wn0 + 32 * j + fr, 0, fh);
        if constexpr (sizeof(T) == 2) __builtin_amdgcn_sched_group_barrier(0x100, FM + FN, 0);
#pragma unroll
        for (int ks = 0; ks < KS; ks++) {
            const int cur = ks & 1, nxt = cur ^ 1;
            if (ks + 1 < KS) {
#pragma unroll
                for (int i = 0; i < FM; i++) af[nxt][i] = read_frag<T>(st, wm0 + 32 * i + fr, ks + 1, fh);
#pragma unroll
                for (int j = 0; j < FN; j++) bfr[nxt][j] = read_frag<T>(st, BM + wn0 + 32 * j + fr, ks + 1, fh);
            }
#pragma unroll
            for (int i = 0; i < FM; i++)
#pragma unroll
                for (int j = 0; j < FN; j++) mma32(acc[i][j], af[cur][i], bfr[cur][j]);
            if constexpr (sizeof(T) == 2) {
                if (ks + 1 < KS) __builtin_amdgcn_sched_group_barrier(0x100, FM + FN, 0);  // DS reads
                __builtin_amdgcn_sched_group_barrier(0x008, FM * FN, 0);                   // MFMAs
            }
        }
    }
#undef GEMM_ISSUE

    if constexpr (F8) {  // per-output-channel weight scales
#pragma unroll
        for (int j = 0; j < FN; j++) {
            const float wsv = a.ws[n0 + wn0 + 32 * j + cl];
#pragma unroll
            for (int i = 0; i < FM; i++)
#pragma unroll
                for (int e = 0; e < 16; e++) acc[i][j][e] *= wsv;
        }
    }

    if constexpr (FUSE_IN) {
        if (a.rstat) {
            // acc = r * acc + (shift W)[vec, col]; every row of the launch has the same
            // modulation vector (checked at launch).
            // The wave's row scales go through its own slot of the (now free) stage buffers;
            // this lane then needs rows 4 (lane / 32) + 32 i + 8 q + 0..3.
            __syncthreads();  // every wave is past its last read of the operand stages
            // In the last slice's stage: the stage after it may hold the QKVG RoPE rows.
            float* rs_lds = reinterpret_cast<float*>(smem + ((nk - 1) % STAGES) * STAGE_BYTES) + wave * WM;
#pragma unroll
            for (int p = 0; p < RPL; p++)
                if (64 * p + lane < WM) rs_lds[64 * p + lane] = rown[p];
            __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): this wave's slot writes landed
            __builtin_amdgcn_wave_barrier();
            float4 rr[FM][4];
#pragma unroll
            for (int i = 0; i < FM; i++)
#pragma unroll
                for (int q = 0; q < 4; q++)
                    rr[i][q] = *reinterpret_cast<const float4*>(rs_lds + 4 * (lane >> 5) + 32 * i + 8 * q);
#pragma unroll
            for (int i = 0; i < FM; i++)
#pragma unroll
                for (int e = 0; e < 16; e++)
#pragma unroll
                    for (int j = 0; j < FN; j++) acc[i][j][e] = acc[i][j][e] * rr[i][e >> 2][e & 3] + bc[j];
        }
    }

    // ---- epilogues (acc layout: see rbase / cl above).
    // Convolution epilogues: per-column bias and, when a Snake output is written, the
    // column's Snake constants (channel col % alpha_n of the alpha block).
    [[maybe_unused]] float bcol[FN], acol[FN], arcol[FN], hcol[FN];
    [[maybe_unused]] const bool snake_out = (EPI == EPI_SNAKE || EPI == EPI_RESUNIT) || a.U != nullptr;
    if constexpr (EPI == EPI_STORE || EPI == EPI_ADD || EPI == EPI_SNAKE || EPI == EPI_RESUNIT) {
#pragma unroll
        for (int j = 0; j < FN; j++) {
            const int col = n0 + wn0 + 32 * j + cl;
            bcol[j] = a.bias ? a.bias[col] : 0.f;
            if (snake_out) {
                const int ch = col % a.alpha_n;
                acol[j] = a.alpha[ch];
                arcol[j] = a.alpha[a.alpha_n + ch];
                hcol[j] = a.alpha[2 * a.alpha_n + ch];
            }
        }
    }
    if constexpr (EPI == EPI_STORE) {
        float* __restrict__ C = a.C;
        T* __restrict__ U = a.U;
#pragma unroll
        for (int i = 0; i < FM; i++)
#pragma unroll
            for (int e = 0; e < 16; e++) {
                int row = rbase + 32 * i + 8 * (e >> 2) + (e & 3);
                if (row >= a.M) continue;
#pragma unroll
                for (int j = 0; j < FN; j++) {
                    const long lin = (long)row * a.N + n0 + wn0 + 32 * j + cl;
                    const float v = acc[i][j][e] + bcol[j];
                    C[lin] = v;
                    if (snake_out && lin >= a.u_lo && lin < a.u_hi)
                        U[lin] = from_f32<T>(snake_eval<T>(v, acol[j], arcol[j], hcol[j]));
                }
            }
    } else if constexpr (EPI == EPI_ADD) {
        // The residual elements of each 32-row block are loaded together before any store:
        // interleaved with the stores to the same array, every load would wait out the
        // memory latency on its own.  (Loading them before the main loop measured slower:
        // the registers and the extra loads compete with the operand stream.)
        float* __restrict__ xg = a.x;
        T* __restrict__ U = a.U;
#pragma unroll
        for (int i = 0; i < FM; i++) {
            float xv[16][FN], rmv[16];
#pragma unroll
            for (int e = 0; e < 16; e++) {
                const int row = rbase + 32 * i + 8 * (e >> 2) + (e & 3);
                const bool ok = row < a.M;
                rmv[e] = ok && a.rmask ? a.rmask[row] : 1.f;
#pragma unroll
                for (int j = 0; j < FN; j++) xv[e][j] = ok ? xg[(long)row * a.N + n0 + wn0 + 32 * j + cl] : 0.f;
            }
#pragma unroll
            for (int e = 0; e < 16; e++) {
                const int row = rbase + 32 * i + 8 * (e >> 2) + (e & 3);
                if (row >= a.M) continue;
#pragma unroll
                for (int j = 0; j < FN; j++) {
                    const long lin = (long)row * a.N + n0 + wn0 + 32 * j + cl;
                    const float v = (xv[e][j] + (acc[i][j][e] + bcol[j])) * rmv[e];
                    xg[lin] = v;
                    if (snake_out) U[lin] = from_f32<T>(snake_eval<T>(v, acol[j], arcol[j], hcol[j]));
                }
            }
        }
    } else if constexpr (EPI == EPI_RESUNIT) {
        // Phase 1: s = Snake(acc + bias) into LDS, slice-major (slice kt2 = columns
        // kt2 * BK .. + BK - 1, BM rows of 128 bytes, chunks swizzled as in the operand
        // stages), while the first W2 slice streams into the slot after it.  Phase 2:
        // acc = s @ W2^T over NK2 slices.  Phase 3: the residual add (+ next Snake).
        // W2 is [BN, K2P] with K2P = BN rounded up to whole slices (zero columns); a partial
        // last slice of the s tile is zero-filled past column BN.
        static_assert(BN % (8 * NW) == 0, "W2 slices split over the waves");
        constexpr int NK2 = (BN + BK - 1) / BK, K2P = NK2 * BK, LPW2 = BN / 8 / NW, EPC = 16 / ES;
        unsigned char* tl = smem;
        unsigned char* w2l = smem + NK2 * BM * 128;
        __syncthreads();  // every wave is done with the main loop's stages
        const __amdgpu_buffer_rsrc_t rW2 = make_rsrc(a.W2, (unsigned)(BN * K2P * ES));
        unsigned voff2[LPW2];
#pragma unroll
        for (int i = 0; i < LPW2; i++) {
            const int r = (wave * LPW2 + i) * 8 + lane / 8;
            voff2[i] = (unsigned)(r * K2P * ES) + (unsigned)swz(r, lane % 8) * 16u;
        }
        if constexpr (K2P != BN) {
            constexpr int c0 = (BN % BK) / EPC;  // first empty chunk of the last slice
            unsigned char* last = tl + (NK2 - 1) * BM * 128;
            for (int idx = threadIdx.x; idx < BM * (8 - c0); idx += 64 * NW) {
                const int r = idx / (8 - c0), c = c0 + idx % (8 - c0);
                *reinterpret_cast<uint4*>(last + r * 128 + (swz(r, c) << 4)) = make_uint4(0u, 0u, 0u, 0u);
            }
        }
#pragma unroll
        for (int i = 0; i < LPW2; i++) buf_load_lds16(rW2, voff2[i], 0u, w2l + (wave * LPW2 + i) * 1024);
#pragma unroll
        for (int i = 0; i < FM; i++)
#pragma unroll
            for (int e = 0; e < 16; e++) {
                const int lr = wm0 + 4 * (lane >> 5) + 32 * i + 8 * (e >> 2) + (e & 3);
#pragma unroll
                for (int j = 0; j < FN; j++) {
                    const int col = wn0 + 32 * j + cl, kt2 = col / BK, kk = col % BK;
                    T* p = reinterpret_cast<T*>(tl + kt2 * BM * 128 + lr * 128 + (swz(lr, kk / EPC) << 4)) + kk % EPC;
                    *p = from_f32<T>(snake_eval<T>(acc[i][j][e] + bcol[j], acol[j], arcol[j], hcol[j]));
                    acc[i][j][e] = 0.f;
                }
            }
#pragma unroll
        for (int kt2 = 0; kt2 < NK2; kt2++) {
            wait_vmcnt<0>();
            __syncthreads();  // W2 slice kt2 has landed; the s tile is complete
            const unsigned char* at = tl + kt2 * BM * 128;
#pragma unroll
            for (int ks = 0; ks < KS; ks++) {
                Frag32<T> af[FM], bf[FN];
#pragma unroll
                for (int i = 0; i < FM; i++) af[i] = read_frag<T>(at, wm0 + 32 * i + fr, ks, fh);
#pragma unroll
                for (int j = 0; j < FN; j++) bf[j] = read_frag<T>(w2l, wn0 + 32 * j + fr, ks, fh);
#pragma unroll
                for (int i = 0; i < FM; i++)
#pragma unroll
                    for (int j = 0; j < FN; j++) mma32(acc[i][j], af[i], bf[j]);
            }
            if (kt2 + 1 < NK2) {
                __syncthreads();  // every wave is done reading the slot
#pragma unroll
                for (int i = 0; i < LPW2; i++)
                    buf_load_lds16(rW2, voff2[i], (unsigned)(kt2 + 1) * 128u, w2l + (wave * LPW2 + i) * 1024);
            }
        }
        float b2[FN], a2[FN], ar2[FN], hc2[FN];
        const bool next = a.U != nullptr;
#pragma unroll
        for (int j = 0; j < FN; j++) {
            const int col = n0 + wn0 + 32 * j + cl;
            b2[j] = a.bias2 ? a.bias2[col] : 0.f;
            if (next) {
                a2[j] = a.alpha2[col];
                ar2[j] = a.alpha2[a.N + col];
                hc2[j] = a.alpha2[2 * a.N + col];
            }
        }
        // The residual in batches of XB rows (loads issued together, then the stores).  Tiles
        // that fit two workgroups per CU take four rows (few registers); the 8-wave 256-row
        // tile runs one workgroup per CU anyway and takes all sixteen (more loads in flight).
        constexpr int XB = BM >= 256 ? 16 : 4;
        float* __restrict__ xg = a.x;
        T* __restrict__ U = a.U;
#pragma unroll
        for (int i = 0; i < FM; i++)
#pragma unroll
            for (int e4 = 0; e4 < 16; e4 += XB) {
                float xv[XB][FN];
#pragma unroll
                for (int e = 0; e < XB; e++) {
                    const int row = rbase + 32 * i + 8 * ((e4 + e) >> 2) + ((e4 + e) & 3);
#pragma unroll
                    for (int j = 0; j < FN; j++)
                        xv[e][j] = row < a.M ? xg[(long)row * a.N + n0 + wn0 + 32 * j + cl] : 0.f;
                }
#pragma unroll
                for (int e = 0; e < XB; e++) {
                    const int row = rbase + 32 * i + 8 * ((e4 + e) >> 2) + ((e4 + e) & 3);
                    if (row >= a.M) continue;
#pragma unroll
                    for (int j = 0; j < FN; j++) {
                        const long lin = (long)row * a.N + n0 + wn0 + 32 * j + cl;
                        const float v = xv[e][j] + (acc[i][j][e4 + e] + b2[j]);
                        xg[lin] = v;
                        if (next) U[lin] = from_f32<T>(snake_eval<T>(v, a2[j], ar2[j], hc2[j]));
                    }
                }
            }
    } else if constexpr (EPI == EPI_SNAKE) {
        T* __restrict__ U = a.U;
#pragma unroll
        for (int i = 0; i < FM; i++)
#pragma unroll
            for (int e = 0; e < 16; e++) {
                const int row = rbase + 32 * i + 8 * (e >> 2) + (e & 3);
                if (row >= a.M) continue;
#pragma unroll
                for (int j = 0; j < FN; j++)
                    U[(size_t)row * a.N + n0 + wn0 + 32 * j + cl] =
                        from_f32<T>(snake_eval<T>(acc[i][j][e] + bcol[j], acol[j], arcol[j], hcol[j]));
            }
    } else if constexpr (EPI == EPI_RESID) {
        // x[row, col] += gate[b(row), col] * C, from the values loaded before the main loop.
        // Fused adaLN producer (Hn set): also Hn = x (1 + scale_next) and the sums of x^2 of
        // each row over the lane group's 32 columns (one half-wave holds one row's 32 columns
        // of a block, so every lane takes part in the reduction; rows past M add zero).
        float* __restrict__ xg = a.x;
        const bool fuse_out = !F8 && a.Hn != nullptr;
        const int np = a.N / 32;
        if (a.S < 32) {  // a 32-row block may span more than two batch rows
            const int step = a.mt.step ? *a.mt.step : 0;
#pragma unroll
            for (int i = 0; i < FM; i++)
#pragma unroll
                for (int e = 0; e < 16; e++) {
                    const int row = rbase + 32 * i + 8 * (e >> 2) + (e & 3);
                    const bool ok = row < a.M;
                    const int b = (ok ? row : a.M - 1) / a.S;
                    const float* g = gate_vec(a.mt, b, a.layer, a.kind, a.N);
                    const float* sc = a.mt.tab + ((size_t)mod_vec_index(a.mt, step, b) * a.mt.layers * 6 +
                                                  (size_t)a.next_layer * 6 + a.next_kind * 3 + 1) * a.N;
#pragma unroll
                    for (int j = 0; j < FN; j++) {
                        const int col = n0 + wn0 + 32 * j + cl;
                        const float xn = ok ? xg[(size_t)row * a.N + col] + g[col] * acc[i][j][e] : 0.f;
                        if (ok) xg[(size_t)row * a.N + col] = xn;
                        if (fuse_out) {
                            if (ok) a.Hn[(size_t)row * a.N + col] = from_f32<T>(xn * (1.f + sc[col]));
                            const float ss = half_wave_sum(xn * xn);
                            if (ok && cl == 0) a.rstat_out[(size_t)row * np + (n0 + wn0) / 32 + j] = ss;
                        }
                    }
                }
        } else {
            // One straight-line body per (all rows inside M, fused output) pair, both uniform
            // per wave: per-element tests would split the stores into separate blocks.
            auto resid_rows = [&](auto full_c, auto fuse_c) {
                constexpr bool FULL = decltype(full_c)::value, FUSE = decltype(fuse_c)::value;
#pragma unroll
                for (int i = 0; i < FM; i++) {
#pragma unroll
                    for (int j = 0; j < FN; j++) {
                        float sq[16];
                        const size_t off0 = (size_t)(rbase + 32 * i) * a.N + n0 + wn0 + 32 * j + cl;
                        float* xr = xg + off0;
                        [[maybe_unused]] T* hr = a.Hn + off0;
#pragma unroll
                        for (int e = 0; e < 16; e++) {
                            const int ro = 8 * (e >> 2) + (e & 3);  // row offset from rbase + 32 i
                            const int row = rbase + 32 * i + ro;
                            const bool ok = FULL || row < a.M;
                            const int u = row >= hi_row[i] ? 1 : 0;
                            const float xn = xpre[i][e][j] + gpre[i][u][j] * acc[i][j][e];
                            sq[e] = ok ? xn * xn : 0.f;
                            if constexpr (FULL) {
                                xr[(size_t)ro * a.N] = xn;
                                if constexpr (FUSE) hr[(size_t)ro * a.N] = from_f32<T>(xn * (1.f + spre[i][u][j]));
                            } else if (ok) {
                                xr[(size_t)ro * a.N] = xn;
                                if constexpr (FUSE) hr[(size_t)ro * a.N] = from_f32<T>(xn * (1.f + spre[i][u][j]));
                            }
                        }
                        if constexpr (FUSE) {
                            // Row sums over the half-wave's 32 columns: a halving butterfly over
                            // lane bits 4..1 (each step keeps half the rows and adds the partner's
                            // values of them), then bit 0; lane l ends with row
                            // e = 8 b4 + 4 b3 + 2 b2 + b1 of l.
                            const int e = half_wave_row_sums(sq, cl);
                            const int row = rbase + 32 * i + 8 * (e >> 2) + (e & 3);
                            if (row < a.M && (cl & 1) == 0) a.rstat_out[(size_t)row * np + (n0 + wn0) / 32 + j] = sq[0];
                        }
                    }
                }
            };
            const bool full = m0 + wm0 + WM <= a.M;
            if (full) {
                if (fuse_out) resid_rows(std::true_type{}, std::true_type{});
                else resid_rows(std::true_type{}, std::false_type{});
            } else {
                if (fuse_out) resid_rows(std::false_type{}, std::true_type{});
                else resid_rows(std::false_type{}, std::false_type{});
            }
        }
    } else if constexpr (EPI == EPI_SWIGLU) {
        // W rows come in 32-row groups alternating W1 / W3 columns: block j even holds
        // u1 and block j+1 the matching u3 for output columns 32 * pair + lane % 32.
        const int half_n = a.N / 2;
        if constexpr (F8) {
            // fp8 output: a pair's 32 columns of a row are one scale block of the next
            // projection's input.  Each wave stages its WM x 32 block of m per pair in its own
            // LDS slot (row stride 33 floats: both passes conflict-free); then lane r owns row
            // r: the block max, the 32 codes as two 16-byte stores, and the scale byte.
            static_assert(WM <= 64, "one staged row per lane");
            constexpr int SLOT = WM * 33 * 4;
            static_assert(STAGES * STAGE_BYTES >= NW * SLOT, "SwiGLU fp8 epilogue needs one LDS slot per wave");
            __syncthreads();  // every wave is past its last read of the operand stages
            float* slot = reinterpret_cast<float*>(smem + wave * SLOT);
#pragma unroll
            for (int j = 0; j < FN; j += 2) {
                const int pair = (n0 + wn0) / 64 + j / 2;
#pragma unroll
                for (int i = 0; i < FM; i++)
#pragma unroll
                    for (int e = 0; e < 16; e++) {
                        const int r = 32 * i + 8 * (e >> 2) + 4 * (lane >> 5) + (e & 3);
                        slot[r * 33 + cl] = silu_f(acc[i][j][e]) * acc[i][j + 1][e];
                    }
                __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): this wave's slot writes landed
                __builtin_amdgcn_wave_barrier();
                if (lane < WM) {
                    float v[32];
                    float amax = 0.f;
#pragma unroll
                    for (int c = 0; c < 32; c++) {
                        v[c] = slot[lane * 33 + c];
                        amax = fmaxf(amax, fabsf(v[c]));
                    }
                    const int ex = mx_exp(amax);
                    const int row = m0 + wm0 + lane;
                    if (row < a.M) {
                        unsigned w[8];
#pragma unroll
                        for (int q = 0; q < 8; q++)
                            w[q] = pack_e4m3(ldexpf(v[4 * q], -ex), ldexpf(v[4 * q + 1], -ex), ldexpf(v[4 * q + 2], -ex),
                                             ldexpf(v[4 * q + 3], -ex));
                        uint4* dst = reinterpret_cast<uint4*>(a.U8 + (size_t)row * half_n + pair * 32);
                        dst[0] = make_uint4(w[0], w[1], w[2], w[3]);
                        dst[1] = make_uint4(w[4], w[5], w[6], w[7]);
                        a.U8s[(size_t)row * (half_n / 32) + pair] = (uint8_t)(127 + ex);
                    }
                }
                __builtin_amdgcn_wave_barrier();  // the slot is rewritten by the next pair
            }
        } else {
            // Straight-line stores when every row of the wave is inside M (uniform).
            auto swiglu_rows = [&](auto full_c) {
                constexpr bool FULL = decltype(full_c)::value;
#pragma unroll
                for (int i = 0; i < FM; i++) {
                    T* ur = a.U + (size_t)(rbase + 32 * i) * half_n + (n0 + wn0) / 2 + cl;
#pragma unroll
                    for (int e = 0; e < 16; e++) {
                        const int ro = 8 * (e >> 2) + (e & 3);
                        if (!FULL && rbase + 32 * i + ro >= a.M) continue;
#pragma unroll
                        for (int j = 0; j < FN; j += 2)
                            ur[(size_t)ro * half_n + 16 * j] = from_f32<T>(silu_f(acc[i][j][e]) * acc[i][j + 1][e]);
                    }
                }
            };
            if (m0 + wm0 + WM <= a.M) swiglu_rows(std::true_type{});
            else swiglu_rows(std::false_type{});
        }
    } else if constexpr (EPI == EPI_CTXKV) {
        // One head (WN = 64 or 128 columns) per wave: region 0 = K (head RMSNorm,
        // norm.rs:60-74, no RoPE), region 1 = V (transposed scatter).  A setup-path
        // epilogue: element stores.  V^T key order: the 32x32x16 attention's (bf16 with
        // 64-dim heads) or the 16x16 attention's (f32, and 128-dim heads).
        constexpr int Dh = WN;
        const int HD = a.H * Dh;
        const int col0 = n0 + wn0;
        const bool is_k = col0 < HD;
        const int h = (is_k ? col0 : col0 - HD) / Dh;
        if (is_k) {
            float nw[FN];
#pragma unroll
            for (int j = 0; j < FN; j++) nw[j] = a.k_norm[h * Dh + 32 * j + cl];
#pragma unroll
            for (int i = 0; i < FM; i++)
#pragma unroll
                for (int e = 0; e < 16; e++) {
                    const int row = rbase + 32 * i + 8 * (e >> 2) + (e & 3);
                    float sq = 0.f;
#pragma unroll
                    for (int j = 0; j < FN; j++) sq += acc[i][j][e] * acc[i][j][e];
                    const float ss = half_wave_sum(sq);
                    const float inv = __builtin_amdgcn_rsqf(ss * (1.f / (float)Dh) + a.eps);
                    if (row >= a.M) continue;
                    T* o = a.Ck + ((size_t)h * a.ctx_stride + a.key_off + row) * Dh;
#pragma unroll
                    for (int j = 0; j < FN; j++) o[32 * j + cl] = from_f32<T>(acc[i][j][e] * inv * nw[j]);
                }
        } else {
#pragma unroll
            for (int i = 0; i < FM; i++)
#pragma unroll
                for (int e = 0; e < 16; e++) {
                    const int row = rbase + 32 * i + 8 * (e >> 2) + (e & 3);
                    if (row >= a.M) continue;
                    const int key = a.key_off + row;
                    const int pos = (sizeof(T) == 2 && Dh == 64) ? vt_pos_bf16(key) : vt_pos_f32(key);
#pragma unroll
                    for (int j = 0; j < FN; j++)
                        a.Cv[((size_t)h * Dh + 32 * j + cl) * a.ctx_vstride + pos] = from_f32<T>(acc[i][j][e]);
                }
        }
    } else if constexpr (EPI == EPI_QKVG && WN == 128) {
        // 128-dim heads (4 x 1 waves: each wave owns 32 rows x one whole head of one region
        // q | k | v | gate).  q / k: head RMSNorm over the 128 columns (norm.rs:60-74), half
        // RoPE on the first H / 2 heads (rope.rs:82-135, interleaved pairs in neighbouring
        // lanes, the (cos, sin) rows read from the table in global memory), q scaled; v:
        // V^T scatter in the 16x16 attention's key order (vt_pos_f32, either dtype); gate:
        // sigmoid.  Element stores: a capability path, not the 64-dim headline path.
        constexpr int Dh = 128;
        const int D = a.D;
        const int col0 = n0 + wn0;
        const int region = col0 / D;
        const int h = (col0 % D) / Dh;
        if (region <= 1) {
            const bool rope = h < a.H / 2;
            const float* nwp = (region == 0 ? a.q_norm : a.k_norm) + h * Dh;
            const float qs = region == 0 ? a.q_scale : 1.f;
            float nw[FN];
#pragma unroll
            for (int j = 0; j < FN; j++) nw[j] = nwp[32 * j + cl] * qs;
            T* dst = region == 0 ? a.Q : a.Kd;
            const float sgn = (cl & 1) ? -1.f : 1.f;
#pragma unroll
            for (int i = 0; i < FM; i++)
#pragma unroll
                for (int e = 0; e < 16; e++) {
                    const int row = rbase + 32 * i + 8 * (e >> 2) + (e & 3);
                    float sq = 0.f;
#pragma unroll
                    for (int j = 0; j < FN; j++) sq += acc[i][j][e] * acc[i][j][e];
                    const float ss = half_wave_sum(sq);
                    const float inv = __builtin_amdgcn_rsqf(ss * (1.f / (float)Dh) + a.eps);
                    int b, sqi;
                    row_bs(row < a.M ? row : a.M - 1, a.S, inv_s, b, sqi);
                    float y[FN];
#pragma unroll
                    for (int j = 0; j < FN; j++) y[j] = acc[i][j][e] * inv * nw[j];
                    if (rope) {
                        // Pair k = 16 j + cl / 2 of token sqi: (y c - y' s, y c + y' s) for the
                        // (even, odd) lane, y' the partner lane's value.
                        const float2* cs = reinterpret_cast<const float2*>(a.rope_cs) + (size_t)sqi * (Dh / 2);
#pragma unroll
                        for (int j = 0; j < FN; j++) {
                            const float2 t = cs[16 * j + (cl >> 1)];
                            const float pr = IRO_DPP(y[j] * sgn, 0xB1) * t.y;
                            y[j] = fmaf(y[j], t.x, pr);
                        }
                    }
                    if (row >= a.M) continue;
                    T* o = dst + (((size_t)b * a.H + h) * a.S + sqi) * Dh;
#pragma unroll
                    for (int j = 0; j < FN; j++) o[32 * j + cl] = from_f32<T>(y[j]);
                }
        } else if (region == 2) {
#pragma unroll
            for (int i = 0; i < FM; i++)
#pragma unroll
                for (int e = 0; e < 16; e++) {
                    const int row = rbase + 32 * i + 8 * (e >> 2) + (e & 3);
                    if (row >= a.M) continue;
                    int b, sqi;
                    row_bs(row, a.S, inv_s, b, sqi);
                    const int pos = vt_pos_f32(sqi);
#pragma unroll
                    for (int j = 0; j < FN; j++)
                        a.Vd[(((size_t)b * a.H + h) * Dh + 32 * j + cl) * a.vt_stride + pos] =
                            from_f32<T>(acc[i][j][e]);
                }
        } else {
#pragma unroll
            for (int i = 0; i < FM; i++)
#pragma unroll
                for (int e = 0; e < 16; e++) {
                    const int row = rbase + 32 * i + 8 * (e >> 2) + (e & 3);
                    if (row >= a.M) continue;
#pragma unroll
                    for (int j = 0; j < FN; j++)
                        a.G[(size_t)row * D + col0 - 3 * D + 32 * j + cl] = from_f32<T>(sigmoid_f(acc[i][j][e]));
                }
        }
    } else if constexpr (EPI == EPI_QKVG) {
        // Each wave owns WM rows x one 64-column head of one region (q | k | v | gate).
        // The stage buffers are free once every wave is past the main loop.  q / k waves read
        // the tile's RoPE rows from the stage after the last slice's (loaded during the last
        // slice) and stage their bf16 tile packed in the last slice's stage (WM x 128 bytes
        // per wave); gate and V waves use a slot of SLOT bytes per wave over both stages: the
        // staged gate tile (stage_off) written out with 16-byte stores, or the V^T transpose
        // (64 x (WM + 2) elements; an odd word stride keeps both passes conflict-free).
        constexpr int VT_BYTES = sizeof(T) == 2 ? 64 * (WM + 2) * 2 : 0;  // f32 scatters V^T directly
        constexpr int SLOT = WM * 256 > VT_BYTES ? WM * 256 : VT_BYTES;
        static_assert(STAGES * STAGE_BYTES >= NW * SLOT, "QKVG epilogue needs one LDS slot per wave");
        const int D = a.D, Dh = 64;
        const int col0 = n0 + wn0;  // first column of this wave's head
        const int region = col0 / D;
        const int h = (col0 % D) / Dh;
        const int half_heads = a.H / 2;
        const int rw0 = m0 + wm0;  // first row of this wave
        const bool rope = region <= 1 && h < half_heads;
        static_assert(NW * WM * 128 <= STAGE_BYTES, "packed q / k staging fits one stage");
        if (rope_wg) asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // this wave's RoPE rows landed
        __syncthreads();
        unsigned char* slot = smem + wave * SLOT;
        if (region <= 1) {
            // Head RMSNorm weight, with the query scale folded in for q.
            const float* nwp = (region == 0 ? a.q_norm : a.k_norm) + h * Dh;
            const float qs = region == 0 ? a.q_scale : 1.f;
            const float nw0 = nwp[cl] * qs, nw1 = nwp[32 + cl] * qs;
            T* dst = region == 0 ? a.Q : a.Kd;
            // RoPE rows of this wave's tokens: [WM][32 pairs][cos, sin].
            const float* rt = reinterpret_cast<const float*>(smem + (nk % STAGES) * STAGE_BYTES) + wm0 * 64;
            unsigned char* qslot = smem + ((nk - 1) % STAGES) * STAGE_BYTES + wave * (WM * 128);
            // Interleaved RoPE pairs (2k, 2k+1) sit in neighbouring lanes: the even lane
            // takes y c - y' s, the odd one y c + y' s (y' the partner's value), so each
            // lane hands its partner its value with the sign the partner needs.
            const float sgn = (cl & 1) ? -1.f : 1.f;
            const int k0 = cl >> 1, k1 = 16 + (cl >> 1);
            // One straight-line body per RoPE setting (the flag is uniform per wave): a
            // runtime test inside the unrolled rows would split them into separate blocks
            // and serialise each row's reduction and table reads.
            auto qk_rows = [&](auto rope_c) {
                constexpr bool ROPE = decltype(rope_c)::value;
#pragma unroll
                for (int i = 0; i < FM; i++)
#pragma unroll
                    for (int e = 0; e < 16; e++) {
                        const int rl = 32 * i + 8 * (e >> 2) + 4 * (lane >> 5) + (e & 3);  // row within the wave
                        const int row = rw0 + rl;
                        const float y0 = acc[i][0][e], y1 = acc[i][1][e];
                        const float ss = half_wave_sum(y0 * y0 + y1 * y1);
                        const float inv = __builtin_amdgcn_rsqf(ss * (1.f / (float)Dh) + a.eps);
                        float ya = y0 * inv * nw0, yb = y1 * inv * nw1;
                        if constexpr (ROPE) {
                            const float2 cs0 = *reinterpret_cast<const float2*>(rt + rl * 64 + 2 * k0);
                            const float2 cs1 = *reinterpret_cast<const float2*>(rt + rl * 64 + 2 * k1);
                            const float pa = IRO_DPP(ya * sgn, 0xB1) * cs0.y;
                            const float pb = IRO_DPP(yb * sgn, 0xB1) * cs1.y;
                            ya = fmaf(ya, cs0.x, pa);
                            yb = fmaf(yb, cs1.x, pb);
                        }
                        if constexpr (sizeof(T) == 2) {
                            acc[i][0][e] = ya;
                            acc[i][1][e] = yb;
                        } else if (row < a.M) {
                            int b, sq;
                            row_bs(row, a.S, inv_s, b, sq);
                            T* o = dst + (((size_t)b * a.H + h) * a.S + sq) * Dh;
                            o[cl] = from_f32<T>(ya);
                            o[32 + cl] = from_f32<T>(yb);
                        }
                    }
            };
            if (rope)
                qk_rows(std::true_type{});
            else
                qk_rows(std::false_type{});
            if constexpr (sizeof(T) == 2) {
                // Staged once every row is computed.
#pragma unroll
                for (int i = 0; i < FM; i++)
#pragma unroll
                    for (int e = 0; e < 16; e++) {
                        const int rl = 32 * i + 8 * (e >> 2) + 4 * (lane >> 5) + (e & 3);
                        *reinterpret_cast<T*>(qslot + stage_off_packed(rl, cl)) = from_f32<T>(acc[i][0][e]);
                        *reinterpret_cast<T*>(qslot + stage_off_packed(rl, 32 + cl)) = from_f32<T>(acc[i][1][e]);
                    }
                // 16-byte stores: 8 lanes per 128-byte head row of [B, H, S, Dh]; pass it
                // writes token row rw0 + 8 it + lane / 8.  All staged reads are issued first.
                const int c = lane & 7;
                uint4 sv[WM / 8];
#pragma unroll
                for (int it = 0; it < WM / 8; it++)
                    sv[it] = *reinterpret_cast<const uint4*>(qslot + stage_off_packed(it * 8 + (lane >> 3), 8 * c));
                if (a.S >= 8 && rw0 + WM <= a.M) {
                    // Every row is inside M: the destination steps by 8 tokens, moving to the
                    // next batch row (H - 1 head blocks further) when the token index wraps.
                    int b, sq;
                    row_bs(rw0 + (lane >> 3), a.S, inv_s, b, sq);
                    T* o = dst + (((size_t)b * a.H + h) * a.S + sq) * Dh + 8 * c;
                    const size_t wrap_add = (size_t)(a.H - 1) * a.S * Dh;
#pragma unroll
                    for (int it = 0; it < WM / 8; it++) {
                        *reinterpret_cast<uint4*>(o) = sv[it];
                        sq += 8;
                        const bool wrap = sq >= a.S;
                        sq = wrap ? sq - a.S : sq;
                        o += 8 * Dh + (wrap ? wrap_add : 0);
                    }
                } else {
#pragma unroll
                    for (int it = 0; it < WM / 8; it++) {
                        const int row = rw0 + it * 8 + (lane >> 3);
                        if (row >= a.M) continue;
                        int b, sq;
                        row_bs(row, a.S, inv_s, b, sq);
                        *reinterpret_cast<uint4*>(dst + (((size_t)b * a.H + h) * a.S + sq) * Dh + 8 * c) = sv[it];
                    }
                }
            }
        } else if (region == 2) {
            // V^T [B,H,Dh,S'] in the key order the attention kernel's A operand wants.
            if constexpr (sizeof(T) == 2) {
                // The wave's WM x 64 block is transposed through LDS, then each lane stores
                // a token pair (s, s+1) — adjacent under the key permutation — as one word.
                constexpr int VS = WM + 2;  // row stride (elements) of the transpose
                T* vt = reinterpret_cast<T*>(slot);  // [64 dims][VS]
#pragma unroll
                for (int i = 0; i < FM; i++)
#pragma unroll
                    for (int e = 0; e < 16; e++) {
                        const int rl = 32 * i + 8 * (e >> 2) + 4 * (lane >> 5) + (e & 3);
#pragma unroll
                        for (int j = 0; j < 2; j++) vt[(32 * j + cl) * VS + rl] = from_f32<T>(acc[i][j][e]);
                    }
                // Pass it covers dims d = it * (64 / PP) + lane / PP of token pair p = lane % PP,
                // the same pair in every pass, so the pair's position and the choice between
                // one word and two elements are decided once per lane.
                constexpr int PP = WM / 2;  // token pairs per wave
                static_assert(64 % PP == 0, "a lane keeps one token pair");
                const int p = lane % PP, row = rw0 + 2 * p;
                if (row < a.M) {
                    int b, sq;
                    row_bs(row, a.S, inv_s, b, sq);
                    // One word only for an even token with its successor in the same batch
                    // row: (s, s+1) are then adjacent and 4-byte aligned under the key
                    // permutation.  With odd S, odd batch rows start on an odd token.
                    if (!(sq & 1) && sq + 1 < a.S && row + 1 < a.M) {
                        T* o = a.Vd + ((size_t)b * a.H + h) * Dh * a.vt_stride + vt_pos_bf16(sq);
#pragma unroll
                        for (int it = 0; it < PP; it++) {
                            const int d = it * (64 / PP) + lane / PP;
                            *reinterpret_cast<unsigned*>(o + (size_t)d * a.vt_stride) =
                                *reinterpret_cast<const unsigned*>(vt + d * VS + 2 * p);
                        }
                    } else {
                        const bool has2 = row + 1 < a.M;
                        int b2 = b, s2 = sq;
                        if (has2) row_bs(row + 1, a.S, inv_s, b2, s2);
                        T* o0 = a.Vd + ((size_t)b * a.H + h) * Dh * a.vt_stride + vt_pos_bf16(sq);
                        T* o1 = a.Vd + ((size_t)b2 * a.H + h) * Dh * a.vt_stride + vt_pos_bf16(s2);
                        for (int it = 0; it < PP; it++) {
                            const int d = it * (64 / PP) + lane / PP;
                            o0[(size_t)d * a.vt_stride] = vt[d * VS + 2 * p];
                            if (has2) o1[(size_t)d * a.vt_stride] = vt[d * VS + 2 * p + 1];
                        }
                    }
                }
            } else {
#pragma unroll
                for (int i = 0; i < FM; i++)
#pragma unroll
                    for (int e = 0; e < 16; e++) {
                        int row = rbase + 32 * i + 8 * (e >> 2) + (e & 3);
                        if (row >= a.M) continue;
                        int b, sq;
                        row_bs(row, a.S, inv_s, b, sq);
                        int pos = vt_pos_f32(sq);
#pragma unroll
                        for (int j = 0; j < 2; j++) {
                            int d = 32 * j + cl;
                            a.Vd[(((size_t)b * a.H + h) * Dh + d) * a.vt_stride + pos] = from_f32<T>(acc[i][j][e]);
                        }
                    }
            }
        } else if constexpr (sizeof(T) == 2) {
            // Gate: sigmoid staged in LDS, then 16-byte stores of the 128-byte row segments.
#pragma unroll
            for (int i = 0; i < FM; i++)
#pragma unroll
                for (int e = 0; e < 16; e++) {
                    const int rl = 32 * i + 8 * (e >> 2) + 4 * (lane >> 5) + (e & 3);
#pragma unroll
                    for (int j = 0; j < 2; j++)
                        *reinterpret_cast<T*>(slot + stage_off(rl, 32 * j + cl)) = from_f32<T>(sigmoid_f(acc[i][j][e]));
                }
            const int c = lane & 7;
            T* gdst = a.G + (col0 - 3 * D) + (size_t)(rw0 + (lane >> 3)) * D + 8 * c;
            uint4 sv[WM / 8];
#pragma unroll
            for (int it = 0; it < WM / 8; it++)
                sv[it] = *reinterpret_cast<const uint4*>(slot + stage_off(it * 8 + (lane >> 3), 8 * c));
            if (rw0 + WM <= a.M) {
#pragma unroll
                for (int it = 0; it < WM / 8; it++) *reinterpret_cast<uint4*>(gdst + (size_t)it * 8 * D) = sv[it];
            } else {
#pragma unroll
                for (int it = 0; it < WM / 8; it++)
                    if (rw0 + it * 8 + (lane >> 3) < a.M) *reinterpret_cast<uint4*>(gdst + (size_t)it * 8 * D) = sv[it];
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

template <typename T, int BM, int BN, int WAVES_M, int WAVES_N, int STAGES, int EPI, bool F8 = false,
          bool CONV = false>
int launch_cfg(const GemmArgs<T>& a, hipStream_t st) {
    constexpr int ES = F8 ? 1 : (int)sizeof(T);
    constexpr int BK = 128 / ES;
    constexpr int kMaxK8 = 8192;  // fp8: the staged block scales take BM * K / 32 bytes of LDS
    if (a.M <= 0 || a.N % BN != 0 || a.K % BK != 0 || a.K <= 0 || (F8 && a.K > kMaxK8)) return -1;
    // Every pointer the instantiation's main loop and epilogue dereference must be set (the
    // guard sits here, under every launcher, so no caller can skip it).
    if (F8 ? (!a.A8 || !a.As || !a.W8 || !a.ws) : (!a.A || !a.W)) return -1;
    const bool snake_out = EPI == EPI_SNAKE || EPI == EPI_RESUNIT || ((EPI == EPI_STORE || EPI == EPI_ADD) && a.U);
    if (snake_out && (!a.alpha || a.alpha_n <= 0)) return -1;
    switch (EPI) {
        case EPI_STORE: if (!a.C) return -1; break;
        case EPI_RESID: if (!a.x || !a.mt.tab) return -1; break;
        case EPI_ADD: if (!a.x) return -1; break;
        case EPI_SWIGLU: if (F8 ? (!a.U8 || !a.U8s) : !a.U) return -1; break;
        case EPI_SNAKE: if (!a.U) return -1; break;
        case EPI_RESUNIT: if (!a.W2 || !a.x || (a.U && !a.alpha2)) return -1; break;
        case EPI_QKVG:
            if (!a.Q || !a.Kd || !a.Vd || !a.G || !a.q_norm || !a.k_norm || !a.rope_cs || a.H <= 0 ||
                a.D != a.H * (BN / WAVES_N) || a.N != 4 * a.D || a.vt_stride < a.S || a.S <= 0)
                return -1;
            break;
        case EPI_CTXKV:
            if (!a.Ck || !a.Cv || !a.k_norm || a.H <= 0 || a.N != 2 * a.H * (BN / WAVES_N)) return -1;
            break;
    }
    // Fused adaLN: a consumer takes bf16 / f32 operands of the QKVG or SwiGLU projections
    // (K a multiple of 32), a producer writes the next operand after a residual update.
    // The consumer loads each row's K / 32 partials as at most 16 float4 (K % 128 == 0, K <= 2048),
    // and every row of the launch shares one modulation vector (the batch rows all map to it).
    if (a.rstat && (F8 || (EPI != EPI_QKVG && EPI != EPI_SWIGLU) || !a.rbias || a.K % 128 || a.K > 2048 ||
                    a.S <= 0 || !a.mt.tab || a.mt.rows_per_vec < (a.M + a.S - 1) / a.S))
        return -1;
    if (a.Hn && (F8 || EPI != EPI_RESID || !a.rstat_out || a.N % 32 || a.next_layer < 0 ||
                 a.next_layer >= a.mt.layers || a.next_kind < 0 || a.next_kind > 1))
        return -1;
    if ((size_t)BN * a.K * ES > 0xffffffffull || (size_t)BM * a.K * ES > 0xffffffffull) return -1;
    if (a.w_tiled && (CONV || BN % 64 != 0)) return -1;
    if (CONV) {
        // conv_cp a multiple of half a slice (a slice straddles at most two taps, at its
        // middle); K = the taps' span rounded up to whole slices.
        if (a.conv_cp <= 0 || a.conv_cp % (BK / 2) != 0 || a.conv_dil <= 0 || a.conv_rows < 0) return -1;
        const size_t taps = (size_t)((a.K + a.conv_cp - 1) / a.conv_cp);
        if ((size_t)a.conv_rows * a.conv_cp * ES > 0xffffffffull ||
            ((size_t)BM + (taps - 1) * a.conv_dil) * a.conv_cp * ES > 0xffffffffull)
            return -1;
    }
    int tiles = ((a.M + BM - 1) / BM) * (a.N / BN);
    // EPI_RESUNIT keeps the Snake'd tile (BN / BK slices of BM rows) and one W2 slice in LDS.
    constexpr int kResLds = EPI == EPI_RESUNIT ? ((BN + BK - 1) / BK) * BM * 128 + BN * 128 : 0;
    constexpr int kStageLds = STAGES * (BM + BN) * 128;
    const size_t lds = (size_t)(kStageLds > kResLds ? kStageLds : kResLds) + (F8 ? (size_t)BM * (a.K / 32) : 0);
    // Per instantiation; the attribute is process-wide.
    static LdsLimit lds_limit;
    constexpr int lds_max = (kStageLds > kResLds ? kStageLds : kResLds) + (F8 ? BM * (kMaxK8 / 32) : 0);
    if (set_lds_limit_once(lds_limit, (const void*)gemm_kernel<T, BM, BN, WAVES_M, WAVES_N, STAGES, EPI, F8, CONV>,
                           lds_max) != hipSuccess)
        return -2;
    gemm_kernel<T, BM, BN, WAVES_M, WAVES_N, STAGES, EPI, F8, CONV><<<tiles, 64 * WAVES_M * WAVES_N, lds, st>>>(a);
    return 0;
}

__global__ __launch_bounds__(256) void tile_rows_kernel(const uint4* __restrict__ src, int N, int nk,
                                                        unsigned char* __restrict__ dst) {
    // One 16-byte chunk per thread, read in row-major order: chunk c of slice kt of row n.
    const long i = (long)blockIdx.x * 256 + threadIdx.x;
    if (i >= (long)N * nk * 8) return;
    const int c = (int)(i % 8);
    const long rk = i / 8;
    const int kt = (int)(rk % nk), n = (int)(rk / nk);
    const size_t off = ((size_t)(n / 64) * nk + kt) * 8192 + (size_t)(n % 64) * 128 + (size_t)c * 16;
    *reinterpret_cast<uint4*>(dst + off) = src[i];
}

}  // namespace

void launch_tile_rows(const void* src, int N, int row_bytes, void* dst, hipStream_t st) {
    const int nk = row_bytes / 128;
    const long chunks = (long)N * nk * 8;
    tile_rows_kernel<<<(unsigned)((chunks + 255) / 256), 256, 0, st>>>(static_cast<const uint4*>(src), N, nk,
                                                                        static_cast<unsigned char*>(dst));
}

// Tile choice per epilogue.  With 2x2 wavefronts of 32x32 blocks the main loop is bound by
// LDS bandwidth (fragment reads + the DMA writes): 1.5x the MFMA time for 128x128 tiles,
// 3x for 64x64.  The wide projections (QKV+gate, W1|W3) use 128x128 tiles in two stages
// (two workgroups per CU); the D-wide projections (Wo, W2) use 64x64 tiles in four stages
// so that N = 1024 still yields enough workgroups (split-K over larger tiles measured
// slower: the f32 partial planes cost more HBM traffic than the LDS time they save), unless
// the batch is large enough for 128x128 tiles.
// Large batches (many utterances) fill the chip with 128x128 tiles too: two full waves of
// workgroups (two per CU) or more.  Tiles are the same MFMA sequence over k in either
// shape, so the choice does not change a single output bit.
template <typename T>
static bool wide_enough(const GemmArgs<T>& a) {
    return a.N % 128 == 0 && (long)((a.M + 127) / 128) * (a.N / 128) >= 512;
}

template <typename T>
int launch_gemm(int epi, const GemmArgs<T>& a, hipStream_t st) {
    if ((epi == EPI_STORE || epi == EPI_ADD) && a.U && (!a.alpha || a.alpha_n <= 0)) return -1;
    switch (epi) {
        case EPI_STORE:
            if (wide_enough(a)) return launch_cfg<T, 128, 128, 2, 2, 2, EPI_STORE>(a, st);
            return launch_cfg<T, 64, 64, 2, 2, 4, EPI_STORE>(a, st);
        case EPI_RESID:
            if (wide_enough(a)) return launch_cfg<T, 128, 128, 2, 2, 2, EPI_RESID>(a, st);
            return launch_cfg<T, 64, 64, 2, 2, 4, EPI_RESID>(a, st);
        case EPI_ADD:
            if (wide_enough(a)) return launch_cfg<T, 128, 128, 2, 2, 2, EPI_ADD>(a, st);
            if (a.N % 128 != 0 && a.N % 192 == 0 && (long)((a.M + 127) / 128) * (a.N / 192) >= 512)
                return launch_cfg<T, 128, 192, 2, 2, 2, EPI_ADD>(a, st);
            return launch_cfg<T, 64, 64, 2, 2, 4, EPI_ADD>(a, st);
        case EPI_SWIGLU: return launch_cfg<T, 128, 128, 2, 2, 2, EPI_SWIGLU>(a, st);
        // QKVG / CTXKV: one head per wave, 2 x 2 waves of 64 columns or 4 x 1 of 128.
        case EPI_QKVG:
            if (a.H > 0 && a.D == a.H * 128) return launch_cfg<T, 128, 128, 4, 1, 2, EPI_QKVG>(a, st);
            return launch_cfg<T, 128, 128, 2, 2, 2, EPI_QKVG>(a, st);
        case EPI_CTXKV:
            if (a.H > 0 && a.N == 2 * a.H * 128) return launch_cfg<T, 128, 128, 4, 1, 2, EPI_CTXKV>(a, st);
            return launch_cfg<T, 128, 128, 2, 2, 2, EPI_CTXKV>(a, st);
    }
    return -1;
}

// fp8 operands: the same tile choices; each 128-byte slice holds 128 k values.
int launch_gemm_fp8(int epi, const GemmArgs<bf16>& a, hipStream_t st) {
    if (!a.A8 || !a.As || !a.W8 || !a.ws || a.K % 128 != 0) return -1;
    switch (epi) {
        case EPI_STORE:
            if (wide_enough(a)) return launch_cfg<bf16, 128, 128, 2, 2, 2, EPI_STORE, true>(a, st);
            return launch_cfg<bf16, 64, 64, 2, 2, 4, EPI_STORE, true>(a, st);
        case EPI_RESID:
            if (wide_enough(a)) return launch_cfg<bf16, 128, 128, 2, 2, 2, EPI_RESID, true>(a, st);
            return launch_cfg<bf16, 64, 64, 2, 2, 4, EPI_RESID, true>(a, st);
        case EPI_SWIGLU: return launch_cfg<bf16, 128, 128, 2, 2, 2, EPI_SWIGLU, true>(a, st);
        case EPI_QKVG: return launch_cfg<bf16, 128, 128, 2, 2, 2, EPI_QKVG, true>(a, st);
    }
    return -1;
}

// Convolutions: the residual streams of the codec decoder are 96 .. 1536 channels (padded
// to 64 / 128) over up to ~10^6 frames, so 128x128 tiles whenever the columns allow.
// Columns that split into 192-wide tiles but not 128-wide ones (a 192-channel stream) use
// 128x192 tiles: 2x2 waves of 64x96, five fragment reads per six MFMAs.
template <typename T>
int launch_gemm_conv(int epi, const GemmArgs<T>& a, hipStream_t st) {
    const bool wide = a.N % 128 == 0, w192 = a.N % 192 == 0, w96 = a.N % 96 == 0;
    if ((epi == EPI_SNAKE || epi == EPI_RESUNIT || (epi != EPI_RESUNIT && a.U)) && (!a.alpha || a.alpha_n <= 0))
        return -1;
    switch (epi) {
        case EPI_STORE:
            // Grids of under 256 128x128 tiles (the stem: 750 frames x 1536 channels over a
            // K of 7168) take 64x64 tiles, four times as many workgroups.
            if (wide && (long)((a.M + 127) / 128) * (a.N / 128) < 256 && a.N % 64 == 0)
                return launch_cfg<T, 64, 64, 2, 2, 4, EPI_STORE, false, true>(a, st);
            if (wide) return launch_cfg<T, 128, 128, 2, 2, 2, EPI_STORE, false, true>(a, st);
            if (w192) return launch_cfg<T, 128, 192, 2, 2, 2, EPI_STORE, false, true>(a, st);
            if (a.N % 64 != 0 && w96) return launch_cfg<T, 256, 96, 4, 1, 2, EPI_STORE, false, true>(a, st);
            return launch_cfg<T, 64, 64, 2, 2, 4, EPI_STORE, false, true>(a, st);
        case EPI_SNAKE:
            if (!a.U) return -1;
            // The largest convolutions (a million frames and more): 256x128 tiles over 8
            // waves halve the weight-tile traffic per output (measured 3-4 % faster there,
            // slower at 90 k frames).
            if (wide && (long)((a.M + 255) / 256) * (a.N / 128) >= 4096)
                return launch_cfg<T, 256, 128, 4, 2, 2, EPI_SNAKE, false, true>(a, st);
            if (wide) return launch_cfg<T, 128, 128, 2, 2, 2, EPI_SNAKE, false, true>(a, st);
            if (w192) return launch_cfg<T, 128, 192, 2, 2, 2, EPI_SNAKE, false, true>(a, st);
            return launch_cfg<T, 64, 64, 2, 2, 4, EPI_SNAKE, false, true>(a, st);
        case EPI_ADD:
            if (wide) return launch_cfg<T, 128, 128, 2, 2, 2, EPI_ADD, false, true>(a, st);
            if (w192) return launch_cfg<T, 128, 192, 2, 2, 2, EPI_ADD, false, true>(a, st);
            return launch_cfg<T, 64, 64, 2, 2, 4, EPI_ADD, false, true>(a, st);
        case EPI_RESUNIT:  // one tile column holds every channel
            if (!a.W2 || !a.x || (a.U && !a.alpha2)) return -1;
            if (a.N == 128 && (long)((a.M + 255) / 256) >= 4096)  // 694 against 777 us at 1.44 M frames
                return launch_cfg<T, 256, 128, 4, 2, 2, EPI_RESUNIT, false, true>(a, st);
            if (a.N == 128) return launch_cfg<T, 128, 128, 2, 2, 2, EPI_RESUNIT, false, true>(a, st);
            if (a.N == 192) return launch_cfg<T, 128, 192, 2, 2, 2, EPI_RESUNIT, false, true>(a, st);
            if (a.N == 96) return launch_cfg<T, 128, 96, 4, 1, 2, EPI_RESUNIT, false, true>(a, st);
            if (a.N == 64) return launch_cfg<T, 64, 64, 2, 2, 4, EPI_RESUNIT, false, true>(a, st);
            return -1;
    }
    return -1;
}

template int launch_gemm_conv<bf16>(int, const GemmArgs<bf16>&, hipStream_t);
template int launch_gemm_conv<float>(int, const GemmArgs<float>&, hipStream_t);
template int launch_gemm<bf16>(int, const GemmArgs<bf16>&, hipStream_t);
template int launch_gemm<float>(int, const GemmArgs<float>&, hipStream_t);

}  // namespace irodori
