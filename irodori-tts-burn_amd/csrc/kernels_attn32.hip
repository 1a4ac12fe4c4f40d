// Joint flash attention for the bf16 model path on the full-rate 32x32x16 matrix-core
// shape (attention.rs:328-425 / :619-664 semantics; a fully masked query row yields 0).
//
// Keys come from two segments read in place — the latent self keys written by the QKV
// GEMM epilogue and the cached text|speaker context keys of the layer — in 64-key tiles.
// Context tiles without a valid key are dropped from the tile list up front.
//
// Per tile and wavefront (32 queries):
//   S'^T = K Q^T - m  10 MFMAs; K tile from LDS (A operand), Q^T in registers (B operand).
//                    The running reference m of every query is subtracted by one more
//                    k16 step per 32-key block: a constant A fragment holding a single 1
//                    (k = 0) against a B fragment holding -m (bf16) at k = 0.  Lane l
//                    ends up holding query l%32 and keys 8a + 4(l/32) + c of every 16-key
//                    group, so a query's max / sum reduce over lanes l and l^32.
//   online softmax   in the log2 domain (Q is pre-scaled by Dh^-1/2 log2 e), with a lazy
//                    reference: m (a bf16 value) moves only on the wavefront's first tile
//                    or when a lane's sum of p = exp2(S') over the tile exceeds 2^TAU, so
//                    the tile max and the O / l rescale are off the common path and
//                    p <= 2^TAU.
//   O^T += V^T P^T   8 MFMAs; P^T is the S'^T accumulator itself, 8 consecutive values per
//                    k16 step, and V^T is stored with bits 2 and 3 of every key index
//                    swapped so that the matching 8 keys are one 16-byte LDS read.
// Workgroup: QB query blocks x KVS key parities; tiles are dealt to the parities
// round-robin and the partial (m, l, O) of the parities are merged through LDS at the
// end.  K and V^T tiles move HBM -> LDS with buffer_load_dwordx4 ... lds (one SGPR
// resource per tile, so rows past the segment end read as zero and need no clamping)
// into unpadded 128-byte rows whose 16-byte chunks are xor-swizzled by (row >> 1) & 7.
// K streams one tile ahead of V so that the score MFMAs of the next tile overlap the
// softmax of the current one.
#include <type_traits>

#include "common.hpp"
#include "kernels.hpp"

namespace irodori {

namespace {

// Max of v over lanes l and l ^ 32 (the two halves of a query column) by v_permlane32_swap,
// a VALU exchange, instead of an LDS-routed shuffle.
__device__ __forceinline__ float max_halves(float v) {
    const unsigned u = __builtin_bit_cast(unsigned, v);
    const auto sw = __builtin_amdgcn_permlane32_swap(u, u, false, false);
    return fmaxf(__builtin_bit_cast(float, (unsigned)sw[0]), __builtin_bit_cast(float, (unsigned)sw[1]));
}
// Sum of v over lanes l and l ^ 32, the same exchange (the same value in both lanes).
__device__ __forceinline__ float sum_halves(float v) {
    const unsigned u = __builtin_bit_cast(unsigned, v);
    const auto sw = __builtin_amdgcn_permlane32_swap(u, u, false, false);
    return __builtin_bit_cast(float, (unsigned)sw[0]) + __builtin_bit_cast(float, (unsigned)sw[1]);
}

typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));

// 8-element operand vector of the 32x32x16 matrix-core step for each element type.
template <typename T>
struct Vec8;
template <>
struct Vec8<bf16> {
    typedef bf16x8 type;
};
template <>
struct Vec8<f16> {
    typedef f16x8 type;
};
__device__ __forceinline__ f32x16 mma32x16(bf16x8 a, bf16x8 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f32x16 mma32x16(f16x8 a, f16x8 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

constexpr int KT = 64;
constexpr int TILE_BYTES = KT * 128;  // 64 rows x 128 bytes (bf16 Dh = 64)
constexpr float TAU = 16.0f;          // lazy-reference slack, log2 units
constexpr float kSumMax = (float)(1u << (int)TAU);  // a lane's tile sum above it moves the reference

__device__ __forceinline__ void raw_barrier() { asm volatile("s_barrier" ::: "memory"); }
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, unsigned bytes) {
    // Raw (stride 0) buffer; dword3 0x00020000 is the gfx9-family data format for raw access.
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}
__device__ __forceinline__ void buf_load_lds16(__amdgpu_buffer_rsrc_t r, unsigned voff, void* lds) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)lds, 16, voff, 0, 0, 0);
}
__device__ __forceinline__ int swz(int r, int c) { return c ^ ((r >> 1) & 7); }
template <typename T>
__device__ __forceinline__ typename Vec8<T>::type frag(const unsigned char* tile, int r, int chunk) {
    return *reinterpret_cast<const typename Vec8<T>::type*>(tile + r * 128 + (swz(r, chunk) << 4));
}
__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }
// x rounded to the operand type (the softmax reference must be exactly representable).
template <typename T>
__device__ __forceinline__ float round_to(float x) { return static_cast<float>(static_cast<T>(x)); }

// Tile list of one (row, head): NT words per lane.  Word w covers the source tiles
// 64 w .. 64 w + 63 (latent tiles first, then context tiles) and holds its active tiles
// compacted to lanes 0 .. cnt_w - 1 as the tile index and its 64-bit key-validity mask;
// list entry i is word w's lane i - base[w] for the last word with base[w] <= i.  Latent
// tiles are valid up to len0 (or carry the host-computed latent mask bits); context tiles
// carry the host-computed bits of the row; tiles without a valid key are dropped.  One word
// (4096 keys) serves every model shape measured here; four words hold 16384 keys.
template <int NT>
struct TileList {
    int t[NT], lo[NT], hi[NT];  // per lane
    int base[NT];               // wave-uniform: list index of word w's first entry
    int nact;                   // wave-uniform
};

// Entry li (wave-uniform, < nact) of one per-lane field of the list.
template <int NT>
__device__ __forceinline__ int tl_read(const int (&v)[NT], const int (&base)[NT], int li) {
    int r = __builtin_amdgcn_readlane(v[0], li & 63);
#pragma unroll
    for (int w = 1; w < NT; w++)
        if (li >= base[w]) r = __builtin_amdgcn_readlane(v[w], (li - base[w]) & 63);
    return r;
}

template <int NT, typename T>
__device__ __forceinline__ TileList<NT> build_tile_list(const AttnArgs<T>& a, int b, int lane, int nt0, int nt1) {
    TileList<NT> tl;
    int total = 0;
#pragma unroll
    for (int w = 0; w < NT; w++) {
        const int g = 64 * w + lane;  // source tile of this lane in word w
        unsigned long long bits = 0ull;
        if (g < nt0) {
            const int rem = a.len0 & (KT - 1);
            bits = a.bits0 ? a.bits0[(size_t)b * nt0 + g] : (g == nt0 - 1 && rem) ? ((1ull << rem) - 1ull) : ~0ull;
        } else if (g < nt0 + nt1) {
            bits = a.bits1[(size_t)b * ((a.stride1 + KT - 1) / KT) + (g - nt0)];
        }
        const bool on = bits != 0ull;
        const unsigned long long act = __ballot(on);
        const int cnt = __popcll(act);
        const int below = __popcll(act & ((1ull << lane) - 1ull));
        // Active lanes go to their rank; the others to distinct slots past the active ones.
        const int dest = 4 * (on ? below : cnt + (lane - below));
        tl.t[w] = __builtin_amdgcn_ds_permute(dest, g);
        tl.lo[w] = __builtin_amdgcn_ds_permute(dest, (int)(unsigned)bits);
        tl.hi[w] = __builtin_amdgcn_ds_permute(dest, (int)(unsigned)(bits >> 32));
        tl.base[w] = total;
        total += cnt;
    }
    tl.nact = total;
    return tl;
}

// S'^T of one 64-key tile (two 32-key blocks): the reference step, then 4 k16 steps.
template <typename T>
__device__ __forceinline__ void score_tile(f32x16 (&s)[2], const unsigned char* kt, int fr, int fh,
                                           const typename Vec8<T>::type (&qf)[4], typename Vec8<T>::type ones,
                                           typename Vec8<T>::type qbias) {
#pragma unroll
    for (int kb = 0; kb < 2; kb++) {
        f32x16 z;
#pragma unroll
        for (int e = 0; e < 16; e++) z[e] = 0.f;
        s[kb] = mma32x16(ones, qbias, z);
    }
    typename Vec8<T>::type kf[2][4];
#pragma unroll
    for (int kb = 0; kb < 2; kb++)
#pragma unroll
        for (int ks = 0; ks < 4; ks++) kf[kb][ks] = frag<T>(kt, 32 * kb + fr, 2 * ks + fh);
#pragma unroll
    for (int kb = 0; kb < 2; kb++)
#pragma unroll
        for (int ks = 0; ks < 4; ks++) s[kb] = mma32x16(kf[kb][ks], qf[ks], s[kb]);
}

// Merge of the KVS key parities' partial (m, l, O) through LDS (the stage buffers, free
// once the caller has synchronised the workgroup): [parity - 1][QB][NB][34][64 lanes].
// Parity p > 0 waves deposit their NB blocks and return false; parity 0 folds them in, in
// parity order, and returns true.  Every wave of the workgroup must call it.
template <int QB, int KVS, int NB>
__device__ __forceinline__ bool merge_parities(unsigned char* smem, int par, int qb, int lane, f32x16 (*o)[2],
                                               float* m_run, float* l_run) {
    float* comb = reinterpret_cast<float*>(smem);
    if (par > 0) {
#pragma unroll
        for (int nb = 0; nb < NB; nb++) {
            float* c = comb + (((size_t)(par - 1) * QB + qb) * NB + nb) * 34 * 64 + lane;
#pragma unroll
            for (int db = 0; db < 2; db++)
#pragma unroll
                for (int e = 0; e < 16; e++) c[(16 * db + e) * 64] = o[nb][db][e];
            c[32 * 64] = m_run[nb];
            c[33 * 64] = l_run[nb];
        }
    }
    __syncthreads();
    if (par > 0) return false;
#pragma unroll
    for (int pp = 1; pp < KVS; pp++)
#pragma unroll
        for (int nb = 0; nb < NB; nb++) {
            const float* c = comb + (((size_t)(pp - 1) * QB + qb) * NB + nb) * 34 * 64 + lane;
            const float m1 = c[32 * 64], l1 = c[33 * 64];
            const float mt = fmaxf(m_run[nb], m1);
            const float mu = mt == -INFINITY ? 0.f : mt;
            const float c0 = fast_exp2(m_run[nb] - mu), c1 = fast_exp2(m1 - mu);
#pragma unroll
            for (int db = 0; db < 2; db++)
#pragma unroll
                for (int e = 0; e < 16; e++) o[nb][db][e] = o[nb][db][e] * c0 + c[(16 * db + e) * 64] * c1;
            l_run[nb] = l_run[nb] * c0 + l1 * c1;
            m_run[nb] = mt;
        }
    return true;
}

// Normalise, gate and store one 32-query block: o[db][e] = O[q][32 db + 8 (e / 4) + 4 fh +
// e % 4] for this lane's query q (lanes l and l ^ 32 hold the two halves of its dims).
// Gate values of one lane's output dims (out_mode 0): dims 32 db + 8 g4 + 4 fh .. + 3.
template <typename T>
struct GateQuads {
    typedef T T4 __attribute__((ext_vector_type(4)));
    T4 v[2][4];
};
template <typename T>
__device__ __forceinline__ void load_gate(const AttnArgs<T>& a, GateQuads<T>& g, int b, int hh, int q, int fh) {
    typedef typename GateQuads<T>::T4 T4;
    q = q < a.Sq ? q : a.Sq - 1;
    const T* gp = a.G + ((size_t)b * a.Sq + q) * (a.H * 64) + hh * 64 + 4 * fh;
#pragma unroll
    for (int db = 0; db < 2; db++)
#pragma unroll
        for (int g4 = 0; g4 < 4; g4++) g.v[db][g4] = *reinterpret_cast<const T4*>(gp + 32 * db + 8 * g4);
}

// gpre: the lane's gate values loaded ahead (out_mode 0), or null to load them here.
template <typename T>
__device__ __forceinline__ void store_block(const AttnArgs<T>& a, const f32x16 (&o)[2], float l_run, int b, int hh,
                                            size_t bh, int q, int fh, const GateQuads<T>* gpre = nullptr) {
    const float l = sum_halves(l_run);
    const float inv = l > 0.f ? 1.f / l : 0.f;
    if (q >= a.Sq) return;
    const size_t m = (size_t)b * a.Sq + q;
    if constexpr (std::is_same<T, bf16>::value) {
        if (a.out_mode == 2) {
            // fp8 operand form: head dims 32 db .. 32 db + 31 of query q are one scale block,
            // split between this lane and lane ^ 32.
            const size_t ob = m * (a.H * 64) + hh * 64;
#pragma unroll
            for (int db = 0; db < 2; db++) {
                float gv[16];
                float amax = 0.f;
#pragma unroll
                for (int g4 = 0; g4 < 4; g4++) {
                    const bf16x4 gt = *reinterpret_cast<const bf16x4*>(a.G + ob + 32 * db + 8 * g4 + 4 * fh);
#pragma unroll
                    for (int c = 0; c < 4; c++) {
                        gv[4 * g4 + c] = o[db][4 * g4 + c] * inv * static_cast<float>(gt[c]);
                        amax = fmaxf(amax, fabsf(gv[4 * g4 + c]));
                    }
                }
                amax = fmaxf(amax, __shfl_xor(amax, 32, 64));
                const int ex = mx_exp(amax);
#pragma unroll
                for (int g4 = 0; g4 < 4; g4++)
                    *reinterpret_cast<unsigned*>(a.O8 + ob + 32 * db + 8 * g4 + 4 * fh) =
                        pack_e4m3(ldexpf(gv[4 * g4], -ex), ldexpf(gv[4 * g4 + 1], -ex), ldexpf(gv[4 * g4 + 2], -ex),
                                  ldexpf(gv[4 * g4 + 3], -ex));
                if (fh == 0) a.O8s[m * (a.H * 2) + hh * 2 + db] = (uint8_t)(127 + ex);
            }
            return;
        }
    }
    // Dims 32 db + 8 g4 + 4 fh .. + 3 of query q.  The output mode is uniform: one
    // straight-line body per mode, the gate loads all issued before the first store.
    if (a.out_mode == 0) {
        typedef typename GateQuads<T>::T4 T4;
        const size_t base = m * (a.H * 64) + hh * 64 + 4 * fh;
        GateQuads<T> gl;
        if (!gpre) load_gate<T>(a, gl, b, hh, q, fh);
        const GateQuads<T>& g = gpre ? *gpre : gl;
#pragma unroll
        for (int db = 0; db < 2; db++)
#pragma unroll
            for (int g4 = 0; g4 < 4; g4++) {
                T4 ov;
#pragma unroll
                for (int c = 0; c < 4; c++)
                    ov[c] = static_cast<T>(o[db][4 * g4 + c] * inv * static_cast<float>(g.v[db][g4][c]));
                *reinterpret_cast<T4*>(a.O + base + 32 * db + 8 * g4) = ov;
            }
    } else {
        float* op = a.Of + ((bh * a.Sq) + q) * 64 + 4 * fh;
#pragma unroll
        for (int db = 0; db < 2; db++)
#pragma unroll
            for (int g4 = 0; g4 < 4; g4++)
                *reinterpret_cast<float4*>(op + 32 * db + 8 * g4) =
                    make_float4(o[db][4 * g4] * inv, o[db][4 * g4 + 1] * inv, o[db][4 * g4 + 2] * inv,
                                o[db][4 * g4 + 3] * inv);
    }
}

// QB query blocks of 32 x KVS key parities = QB*KVS wavefronts per workgroup.
// Workgroup id -> (query block, head, row) with the query block fastest and the
// XCD-aware remap on top, so each XCD keeps whole (row, head) K/V sets in its L2.
//
// Software pipeline per wavefront: while the softmax of tile j runs on the VALU, the
// score MFMAs of tile j + 1 run on the matrix core (interleaved by scheduling groups),
// then P_j V_j.  K therefore streams one tile ahead of V: at the barrier of iteration j
// the K tiles of iteration j + 1 and the V tiles of iteration j have landed, and the
// loads of K_{j+2} / V_{j+1} are issued into the slots freed by iteration j - 1.  LDS:
// K ring [2][KVS] tiles + V ring [2][KVS] tiles.
template <typename T, int QB, int KVS, int NT>
// At most two wavefronts per SIMD (the 64 KB of LDS allows no more): the register budget
// that buys lets every fragment read of a tile go out before the MFMAs that consume it.
__global__ __launch_bounds__(64 * QB * KVS) __attribute__((amdgpu_waves_per_eu(1, 2))) void attn32_kernel(
    AttnArgs<T> a, int nqb) {
    typedef typename Vec8<T>::type V8;
    constexpr int NW = QB * KVS;
    constexpr int LPK = KVS * 8 / NW;  // load instructions per wave per K (or V) stage
    static_assert(LPK * NW == KVS * 8, "tiles must split over the waves");
    static_assert((KVS - 1) * QB * 34 * 64 * 4 <= 4 * KVS * TILE_BYTES, "merge buffer must fit the rings");
    extern __shared__ __attribute__((aligned(1024))) unsigned char smem[];
    unsigned char* kring = smem;                        // [2][KVS][TILE_BYTES]
    unsigned char* vring = smem + 2 * KVS * TILE_BYTES;  // [2][KVS][TILE_BYTES]

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int qb = wave % QB, par = wave / QB;
    const int pid = xcd_remap(blockIdx.x, gridDim.x);
    const int qblk = pid % nqb, bhid = pid / nqb;
    const int hh = bhid % a.H, b = bhid / a.H;
    const int q0 = qblk * (32 * QB) + 32 * qb;
    const int fr = lane & 31, fh = lane >> 5;
    const size_t bh = (size_t)b * a.H + hh;

    const int nt0 = (a.len0 + KT - 1) / KT;
    const int nt1 = a.K1 ? (a.len1 + KT - 1) / KT : 0;
    const TileList<NT> tl = build_tile_list<NT>(a, b, lane, nt0, nt1);
    const int nact = tl.nact;
    const int niter = (nact + KVS - 1) / KVS;

    const T* K0b = a.K0 + bh * a.stride0 * 64;
    const T* K1b = a.K1 ? a.K1 + bh * a.stride1 * 64 : nullptr;
    const T* V0b = a.V0 + bh * 64 * (size_t)a.vstride0;
    const T* V1b = a.V1 ? a.V1 + bh * 64 * (size_t)a.vstride1 : nullptr;

    // Load instruction ii of this wave within a K (or V) stage: gi = wave*LPK + ii ->
    // parity tile gi / 8, rows 8 (gi % 8) .. +7; lane -> row + lane / 8, physical chunk
    // lane % 8.  The lane byte offsets are fixed per ii (and per segment for V^T rows).
    unsigned voK[LPK], voV0[LPK], voV1[LPK];
#pragma unroll
    for (int ii = 0; ii < LPK; ii++) {
        const int gi = wave * LPK + ii;
        const int r = (gi % 8) * 8 + lane / 8;
        const unsigned cb = (unsigned)swz(r, lane % 8) * 16u;
        voK[ii] = (unsigned)r * 128u + cb;
        voV0[ii] = (unsigned)r * (unsigned)a.vstride0 * 2u + cb;
        voV1[ii] = (unsigned)r * (unsigned)a.vstride1 * 2u + cb;
    }

    // Issue the K (kind 0) or V^T (kind 1) tiles of iteration j into ring slot sl: tile
    // list entries j*KVS + p, clamped to the last entry so every wave issues LPK loads.
#define ATT_ISSUE(kind_, j_, sl_)                                                             \
    do {                                                                                      \
        _Pragma("unroll") for (int ii = 0; ii < LPK; ii++) {                                  \
            const int gi = wave * LPK + ii;                                                   \
            int li = (j_) * KVS + gi / 8;                                                     \
            li = li < nact ? li : nact - 1;                                                   \
            const int t = tl_read<NT>(tl.t, tl.base, li);                                     \
            const bool s0 = t < nt0;                                                          \
            const int key0 = s0 ? t * KT : (t - nt0) * KT;                                    \
            unsigned char* dst = ((kind_) ? vring : kring) + ((sl_) * KVS + gi / 8) * TILE_BYTES + (gi % 8) * 1024; \
            if ((kind_) == 0) {                                                               \
                const int len = s0 ? a.len0 : a.len1;                                         \
                buf_load_lds16(make_rsrc((s0 ? K0b : K1b) + (size_t)key0 * 64, (unsigned)(len - key0) * 128u), \
                               voK[ii], dst);                                                 \
            } else {                                                                          \
                const int vs = s0 ? a.vstride0 : a.vstride1;                                  \
                buf_load_lds16(make_rsrc((s0 ? V0b : V1b) + key0, (unsigned)(64 * vs - key0) * 2u), \
                               s0 ? voV0[ii] : voV1[ii], dst);                                \
            }                                                                                 \
        }                                                                                     \
    } while (0)

    // Q^T fragments (B operand): query q0 + fr, dims 16 ks + 8 fh .. +8.
    V8 qf[4];
    {
        int q = q0 + fr;
        q = q < a.Sq ? q : a.Sq - 1;
        const T* qp = a.Q + (bh * a.Sq + q) * 64 + 8 * fh;
#pragma unroll
        for (int ks = 0; ks < 4; ks++) qf[ks] = *reinterpret_cast<const V8*>(qp + 16 * ks);
    }
    // Reference subtraction fragments: A = 1 at k = 0 for every key row, B = -m at k = 0.
    V8 ones, qbias;
#pragma unroll
    for (int e = 0; e < 8; e++) {
        ones[e] = static_cast<T>(0.f);
        qbias[e] = static_cast<T>(0.f);
    }
    if (fh == 0) ones[0] = static_cast<T>(1.f);

    f32x16 o[2];
#pragma unroll
    for (int db = 0; db < 2; db++)
#pragma unroll
        for (int e = 0; e < 16; e++) o[db][e] = 0.f;
    float m_ref = 0.f, l_run = 0.f;
    bool first = true;  // wave-uniform: no tile processed yet

    // Prologue: K_0, V_0, then K_1 in flight; scores of tile 0.  A (row, head) with no
    // valid key at all (nact = 0, the same for every wave of the workgroup) issues no load
    // (the clamped tile index would be -1) and runs no iteration: its queries store 0.
    f32x16 s[2];
    if (nact > 0) {
        ATT_ISSUE(0, 0, 0);
        ATT_ISSUE(1, 0, 0);
        if (niter > 1) {
            ATT_ISSUE(0, 1, 1);
            asm volatile("s_waitcnt vmcnt(%0)" ::"n"(LPK) : "memory");
        } else {
            asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        }
        raw_barrier();
        if (par < nact) score_tile<T>(s, kring + par * TILE_BYTES, fr, fh, qf, ones, qbias);
    }

    // Two tiles per iteration with the score buffers swapping roles (no copy of the next
    // tile's scores into the current ones).  Tile step j consumes sc (tile j's scores) and
    // leaves tile j + 1's scores in sn.
    f32x16 sn[2];
    // FIRST: the wavefront's first tile (j = 0), whose reference comes from the tile's own
    // max before any exponential (the later tiles move it only when their sums overflow).
    auto tile_step = [&](auto first_c, const int j, f32x16 (&sc)[2], f32x16 (&sn)[2]) {
        constexpr bool FIRST = decltype(first_c)::value;
        // K_{j+1} and V_j have landed once this wave's loads are done and all waves met.
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        raw_barrier();
        if (j + 1 < niter) ATT_ISSUE(1, j + 1, (j + 1) & 1);
        if (j + 2 < niter) ATT_ISSUE(0, j + 2, j & 1);
        const int li = j * KVS + par;
        if (li >= nact) return;  // this parity has no tile in the last iteration
        // V^T fragments of tile j, read now so that their latency hides behind the softmax.
        const unsigned char* vt = vring + ((j & 1) * KVS + par) * TILE_BYTES;
        V8 vf[2][4];
#pragma unroll
        for (int db = 0; db < 2; db++)
#pragma unroll
            for (int g = 0; g < 4; g++) vf[db][g] = frag<T>(vt, 32 * db + fr, 2 * g + fh);

        // Mask (partial tiles only): keys 32 kb + 8 g4 + 4 fh + c of this lane.
        const unsigned vlo = (unsigned)tl_read<NT>(tl.lo, tl.base, li);
        const unsigned vhi = (unsigned)tl_read<NT>(tl.hi, tl.base, li);
        if ((vlo & vhi) != 0xffffffffu) {
#pragma unroll
            for (int kb = 0; kb < 2; kb++) {
                const unsigned w = (kb ? vhi : vlo) >> (4 * fh);
#pragma unroll
                for (int g4 = 0; g4 < 4; g4++)
#pragma unroll
                    for (int c = 0; c < 4; c++)
                        if (!((w >> (8 * g4 + c)) & 1u)) sc[kb][4 * g4 + c] = -INFINITY;
            }
        }
        // Softmax of tile j against the current reference, on the VALU, while the scores
        // of tile j + 1 run on the matrix core.  (Those are computed unconditionally to keep
        // one scheduling region; without a next tile the slot holds stale data and the
        // result is dropped.)  The wavefront's first tile sets the reference from its max
        // before the exponentials; later tiles correct it afterwards, off the common path,
        // only when a lane's sum shows a probability that may exceed 2^TAU (any p > 2^TAU
        // makes the sum exceed it; an overflow to +inf does too).
        // The next tile's scores subtract the reference in use now (qbias is updated below),
        // so a moved reference also shifts the scores already computed into sn.
        if constexpr (FIRST) {
            // The reference is the tile max (rounded to T; both key halves of a query), taken
            // before the exponentials and before the next tile's scores, which then subtract
            // it inside their MFMAs like every later tile's; O and l are still zero.
            float m16[16];
#pragma unroll
            for (int e = 0; e < 16; e++) m16[e] = fmaxf(sc[0][e], sc[1][e]);
#pragma unroll
            for (int w = 8; w > 0; w >>= 1)
#pragma unroll
                for (int e = 0; e < w; e++) m16[e] = fmaxf(m16[e], m16[e + w]);
            m_ref = round_to<T>(max_halves(m16[0]));
#pragma unroll
            for (int kb = 0; kb < 2; kb++)
#pragma unroll
                for (int e = 0; e < 16; e++) sc[kb][e] -= m_ref;
            if (fh == 0) qbias[0] = static_cast<T>(-m_ref);
        }
        score_tile<T>(sn, kring + (((j + 1) & 1) * KVS + par) * TILE_BYTES, fr, fh, qf, ones, qbias);
        float psum = 0.f;
        V8 pf[4];
#pragma unroll
        for (int kb = 0; kb < 2; kb++)
#pragma unroll
            for (int e = 0; e < 16; e++) {
                const float p = fast_exp2(sc[kb][e]);
                psum += p;
                pf[2 * kb + (e >> 3)][e & 7] = static_cast<T>(p);
            }
        // 8 K-fragment reads, then each score MFMA followed by a slice of the softmax.
        __builtin_amdgcn_sched_group_barrier(0x100, 8, 0);
#pragma unroll
        for (int i = 0; i < 10; i++) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
            __builtin_amdgcn_sched_group_barrier(0x002, 8, 0);
        }
        const unsigned long long over = FIRST ? 0ull : __ballot(!(psum <= kSumMax));
        if (over) {
            // Lanes l and l ^ 32 hold one query's two key halves: either one asks for both.
            const bool need = ((over >> lane) | (over >> (lane ^ 32))) & 1ull;
            // Tile max as a balanced tree, then the halves.
            float m16[16];
#pragma unroll
            for (int e = 0; e < 16; e++) m16[e] = fmaxf(sc[0][e], sc[1][e]);
#pragma unroll
            for (int w = 8; w > 0; w >>= 1)
#pragma unroll
                for (int e = 0; e < w; e++) m16[e] = fmaxf(m16[e], m16[e + w]);
            const float mx = max_halves(m16[0]);
            const float nref = need ? round_to<T>(m_ref + mx) : m_ref;
            const float delta = nref - m_ref;
            const float corr = fast_exp2(-delta);
            m_ref = nref;
#pragma unroll
            for (int db = 0; db < 2; db++) o[db] *= corr;
            l_run *= corr;
            psum = 0.f;
#pragma unroll
            for (int kb = 0; kb < 2; kb++)
#pragma unroll
                for (int e = 0; e < 16; e++) {
                    sc[kb][e] -= delta;
                    sn[kb][e] -= delta;
                    const float p = fast_exp2(sc[kb][e]);
                    psum += p;
                    pf[2 * kb + (e >> 3)][e & 7] = static_cast<T>(p);
                }
            if (fh == 0) qbias[0] = static_cast<T>(-m_ref);
        }
        first = false;
        l_run += psum;
        // O^T += V^T P^T over the 4 16-key groups of the tile.
#pragma unroll
        for (int db = 0; db < 2; db++)
#pragma unroll
            for (int g = 0; g < 4; g++) o[db] = mma32x16(vf[db][g], pf[g], o[db]);
    };
    if (niter > 0) tile_step(std::true_type{}, 0, s, sn);
    for (int j = 1; j < niter; j += 2) {
        tile_step(std::false_type{}, j, sn, s);
        if (j + 1 < niter) tile_step(std::false_type{}, j + 1, s, sn);
    }
#undef ATT_ISSUE
    float m_run = first ? -INFINITY : m_ref;

    // Merge the KVS parities through LDS (reusing the stage buffers; every load has
    // landed since the last iteration waits for all of them), then normalise, gate, store.
    if constexpr (KVS > 1) {
        __syncthreads();
        if (!merge_parities<QB, KVS, 1>(smem, par, qb, lane, &o, &m_run, &l_run)) return;
    }
    store_block<T>(a, o, l_run, b, hh, bh, q0 + fr, fh);
}

template <typename T, int QB, int KVS, int NT>
int launch_attn32_cfg(const AttnArgs<T>& a, hipStream_t st) {
    const size_t lds = (size_t)4 * KVS * TILE_BYTES;
    static LdsLimit lds_limit;
    if (set_lds_limit_once(lds_limit, (const void*)attn32_kernel<T, QB, KVS, NT>, (int)lds) != hipSuccess)
        return -2;
    const int nqb = (a.Sq + 32 * QB - 1) / (32 * QB);
    attn32_kernel<T, QB, KVS, NT><<<dim3(nqb * a.H * a.B), 64 * QB * KVS, lds, st>>>(a, nqb);
    return 0;
}

template <typename T>
int launch_attention32_t(const AttnArgs<T>& a, hipStream_t st) {
    if (a.Sq <= 0 || a.len0 <= 0 || !a.v_transposed || !a.prescaled || (a.mask0 && !a.bits0)) return -1;
    if (a.K1 && !a.bits1) return -1;
    if ((a.vstride0 % KT) || (a.K1 && (a.vstride1 % KT))) return -1;
    if (!std::is_same<T, bf16>::value && a.out_mode == 2) return -1;
    const int ntiles = (a.len0 + KT - 1) / KT + (a.K1 ? (a.len1 + KT - 1) / KT : 0);
    if (ntiles > kAttnMaxKeyTiles) return -1;  // four tile-list words per lane (16384 keys)
    // 2 query blocks x 2 key parities (4 waves, 64 KB LDS) at every size.  Against 4 x 2:
    // one CFG row of 750 frames 18.2 vs 21.1 us with context keys, 12.3 vs 14.5 us without;
    // B = 2 rows 42.0 vs 42.2 us per operator call; BASELINE config 5 (32 rows) 340.5 vs
    // 344.4 ms per RF run.  Every query block's arithmetic is the same in either shape (its
    // two parities merged in the same order), so the shape never changes an output bit.
    // One key parity (4 x 1, 32 KB) ran config 5 faster still (323.8 ms) but slower at
    // B = 2 (45.2 us), and a size-dependent choice would make a row's result depend on the
    // batch it is launched with.
    // The tile list of up to 4096 keys fits one word per lane; longer key ranges take four
    // (the same arithmetic per tile, in the same order).
    if (ntiles <= 64) return launch_attn32_cfg<T, 2, 2, 1>(a, st);
    return launch_attn32_cfg<T, 2, 2, 4>(a, st);
}

// Operator staging (irodori_op_sdpa, Dh = 64 on 16-bit operands): the caller's Q, V and
// float key mask in the layouts attn32_kernel reads.  One block per (row, head) and
// 64-key tile: Q rows pre-scaled by scale * log2(e) (rounded once more to T), the tile's
// V rows transposed through LDS into V^T rows in vt_pos_bf16 key order (keys past seq_kv
// zero), and the tile's 64-bit key-validity word (key < seq_kv and mask >= 0.5; the
// mask is per batch row, so only head 0 writes it).
template <typename T>
__global__ __launch_bounds__(256) void sdpa_stage_kernel(const T* __restrict__ q, const T* __restrict__ v,
                                                         const float* __restrict__ mask, int H, int Sq, int Skv,
                                                         int vstride, float qmul, T* __restrict__ qs,
                                                         T* __restrict__ vt, unsigned long long* __restrict__ bits) {
    __shared__ T tile[64][64 + 2];
    const int t = blockIdx.x, bh = blockIdx.y, b = bh / H, h = bh % H;
    const int ntq = (Sq + 63) / 64, ntk = vstride / 64;
    const int tid = threadIdx.x;
    if (t < ntq) {  // 64 query rows of 64 dims
        const size_t base = ((size_t)bh * Sq + (size_t)t * 64) * 64;
        const int rows = Sq - t * 64 < 64 ? Sq - t * 64 : 64;
        for (int i = tid; i < rows * 64; i += 256) qs[base + i] = static_cast<T>(static_cast<float>(q[base + i]) * qmul);
    }
    if (t >= ntk) return;
    const int k0 = t * 64;
    for (int i = tid; i < 64 * 64; i += 256) {
        const int kk = i / 64, d = i % 64, key = k0 + kk;
        tile[kk][d] = key < Skv ? v[((size_t)bh * Skv + key) * 64 + d] : static_cast<T>(0.f);
    }
    __syncthreads();
    for (int i = tid; i < 64 * 64; i += 256) {
        const int d = i / 64, kk = i % 64;
        vt[((size_t)bh * 64 + d) * vstride + vt_pos_bf16(k0 + kk)] = tile[kk][d];
    }
    if (h == 0 && tid < 64) {
        const int key = k0 + tid;
        const bool ok = key < Skv && (mask == nullptr || mask[(size_t)b * Skv + key] >= 0.5f);
        const unsigned long long w = __ballot(ok);
        if (tid == 0) bits[(size_t)b * ntk + t] = w;
    }
}

}  // namespace

int launch_attention32(const AttnArgs<bf16>& a, hipStream_t st) { return launch_attention32_t<bf16>(a, st); }
int launch_attention32(const AttnArgs<f16>& a, hipStream_t st) { return launch_attention32_t<f16>(a, st); }

size_t sdpa_stage_bytes(int B, int H, int Sq, int Skv) {
    const size_t vs = (size_t)(Skv + 63) / 64 * 64;
    auto al = [](size_t n) { return (n + 255) / 256 * 256; };
    return al((size_t)B * H * Sq * 64 * 2) + al((size_t)B * H * 64 * vs * 2) + al((size_t)B * (vs / 64) * 8);
}

template <typename T>
int launch_sdpa_staged(const T* q, const T* k, const T* v, const float* mask, int B, int H, int Sq, int Skv,
                       float scale, float* out, void* ws, size_t ws_bytes, hipStream_t st) {
    const int vs = (Skv + 63) / 64 * 64;
    if (B <= 0 || H <= 0 || Sq <= 0 || Skv <= 0 || vs / 64 > kAttnMaxKeyTiles) return -1;
    if (ws_bytes < sdpa_stage_bytes(B, H, Sq, Skv) || ((uintptr_t)ws & 255)) return -1;
    auto al = [](size_t n) { return (n + 255) / 256 * 256; };
    unsigned char* p = static_cast<unsigned char*>(ws);
    T* qs = reinterpret_cast<T*>(p);
    T* vt = reinterpret_cast<T*>(p + al((size_t)B * H * Sq * 64 * 2));
    unsigned long long* bits =
        reinterpret_cast<unsigned long long*>(p + al((size_t)B * H * Sq * 64 * 2) + al((size_t)B * H * 64 * vs * 2));
    const int ntq = (Sq + 63) / 64, ntk = vs / 64;
    sdpa_stage_kernel<T><<<dim3(ntq > ntk ? ntq : ntk, B * H), 256, 0, st>>>(
        q, v, mask, H, Sq, Skv, vs, scale * 1.4426950408889634f, qs, vt, bits);
    AttnArgs<T> a{};
    a.Q = qs;
    a.K0 = k;
    a.V0 = vt;
    a.len0 = Skv;
    a.stride0 = Skv;
    a.bits0 = bits;
    a.B = B;
    a.H = H;
    a.Sq = Sq;
    a.scale = scale;
    a.v_transposed = true;
    a.prescaled = true;
    a.vstride0 = vs;
    a.out_mode = 1;
    a.Of = out;
    return launch_attention32_t<T>(a, st);
}
template int launch_sdpa_staged<bf16>(const bf16*, const bf16*, const bf16*, const float*, int, int, int, int, float,
                                      float*, void*, size_t, hipStream_t);
template int launch_sdpa_staged<f16>(const f16*, const f16*, const f16*, const float*, int, int, int, int, float,
                                     float*, void*, size_t, hipStream_t);

}  // namespace irodori
