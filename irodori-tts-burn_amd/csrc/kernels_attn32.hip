// Joint flash attention for the bf16 model path on the full-rate 32x32x16 matrix-core
// shape (attention.rs:328-425 / :619-664 semantics; a fully masked query row yields 0).
//
// Keys come from two segments read in place — the latent self keys written by the QKV
// GEMM epilogue and the cached text|speaker context keys of the layer — in 64-key tiles.
// Context tiles without a valid key are dropped from the tile list up front.
//
// Per tile and wavefront (32 queries):
//   S^T = K Q^T      8 MFMAs; K tile from LDS (A operand), Q^T in registers (B operand).
//                    Lane l ends up holding query l%32 and keys 8a + 4(l/32) + c of every
//                    16-key group, so a query's max / sum reduce over lanes l and l^32.
//   online softmax   in the log2 domain (Q is pre-scaled by Dh^-1/2 log2 e).
//   O^T += V^T P^T   8 MFMAs; P^T is the S^T accumulator itself, 8 consecutive values per
//                    k16 step, and V^T is stored with bits 2 and 3 of every key index
//                    swapped so that the matching 8 keys are one 16-byte LDS read.
// Workgroup: QB query blocks x KVS key parities = 4 wavefronts; tiles are dealt to the
// parities round-robin and the partial (m, l, O) of the two parities are merged through
// LDS at the end.  K and V^T tiles move HBM -> LDS with global_load_lds_dwordx4 into
// unpadded 128-byte rows whose 16-byte chunks are xor-swizzled by (row >> 1) & 7, double
// buffered, with raw barriers so the next tile's loads stay in flight.
#include "common.hpp"
#include "kernels.hpp"

namespace irodori {

namespace {

typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));

constexpr int KT = 64;
constexpr int TILE_BYTES = KT * 128;  // 64 rows x 128 bytes (bf16 Dh = 64)

__device__ __forceinline__ void raw_barrier() { asm volatile("s_barrier" ::: "memory"); }
__device__ __forceinline__ void load_lds16(const void* g, void* lds) {
    __builtin_amdgcn_global_load_lds(g, (__attribute__((address_space(3))) void*)lds, 16, 0, 0);
}
__device__ __forceinline__ int swz(int r, int c) { return c ^ ((r >> 1) & 7); }
__device__ __forceinline__ bf16x8 frag(const unsigned char* tile, int r, int chunk) {
    return *reinterpret_cast<const bf16x8*>(tile + r * 128 + (swz(r, chunk) << 4));
}
__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// Tile list of one (row, head): entry i < nact of the list is held by lane i as the tile
// index and its 64-bit key-validity mask.  Latent tiles are valid up to len0; context
// tiles carry the host-computed bits of the row and tiles without a valid key are dropped.
struct TileList {
    int t, lo, hi;  // per lane
    int nact;       // wave-uniform
};

__device__ __forceinline__ TileList build_tile_list(const AttnArgs<bf16>& a, int b, int lane, int nt0, int nt1) {
    unsigned long long bits = 0ull;
    if (lane < nt0) {
        const int rem = a.len0 & (KT - 1);
        bits = (lane == nt0 - 1 && rem) ? ((1ull << rem) - 1ull) : ~0ull;
    } else if (lane < nt0 + nt1) {
        bits = a.bits1[(size_t)b * ((a.stride1 + KT - 1) / KT) + (lane - nt0)];
    }
    const bool on = bits != 0ull;
    const unsigned long long act = __ballot(on);
    TileList tl;
    tl.nact = __popcll(act);
    const int below = __popcll(act & ((1ull << lane) - 1ull));
    // Active lanes go to their rank; the others to distinct slots past the active ones.
    const int dest = 4 * (on ? below : tl.nact + (lane - below));
    tl.t = __builtin_amdgcn_ds_permute(dest, lane);
    tl.lo = __builtin_amdgcn_ds_permute(dest, (int)(unsigned)bits);
    tl.hi = __builtin_amdgcn_ds_permute(dest, (int)(unsigned)(bits >> 32));
    return tl;
}

// QB query blocks of 32 x KVS key parities = QB*KVS wavefronts per workgroup, ST-stage
// HBM -> LDS pipeline.  Workgroup id -> (query block, head, row) with the query block
// fastest and the XCD-aware remap on top, so each XCD keeps whole (row, head) K/V sets
// in its L2.
template <int QB, int KVS, int ST>
__global__ __launch_bounds__(64 * QB * KVS) void attn32_kernel(AttnArgs<bf16> a, int nqb) {
    constexpr int NW = QB * KVS;
    constexpr int STAGE_BYTES = KVS * 2 * TILE_BYTES;
    constexpr int LPW = KVS * 2 * 8 / NW;  // load instructions per wave per stage
    static_assert(LPW * NW == KVS * 2 * 8, "tiles must split over the waves");
    static_assert((KVS - 1) * QB * 34 * 64 * 4 <= ST * STAGE_BYTES, "merge buffer must fit the stages");
    extern __shared__ __attribute__((aligned(1024))) unsigned char smem[];

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
    const TileList tl = build_tile_list(a, b, lane, nt0, nt1);
    const int nact = tl.nact;
    const int niter = (nact + KVS - 1) / KVS;

    const bf16* K0b = a.K0 + bh * a.stride0 * 64;
    const bf16* K1b = a.K1 ? a.K1 + bh * a.stride1 * 64 : nullptr;
    const bf16* V0b = a.V0 + bh * 64 * (size_t)a.vstride0;
    const bf16* V1b = a.V1 ? a.V1 + bh * 64 * (size_t)a.vstride1 : nullptr;

    // Issue the loads of iteration j into stage buffer sb: tile list entries j*KVS + p
    // (clamped to the last entry, so every wave issues LPW loads per stage).  Instruction
    // ii of this wave: gi = wave*LPW + ii -> tile slot gi / 8 = 2 p + kind (kind 0 = K
    // rows = keys, kind 1 = V^T rows = dims), rows 8 (gi % 8) .. +7, lane -> row
    // + lane / 8, physical chunk lane % 8.  Everything but the lane part is wave-uniform.
#define ATT_ISSUE(j_, sb_)                                                                    \
    do {                                                                                      \
        _Pragma("unroll") for (int ii = 0; ii < LPW; ii++) {                                  \
            const int gi = wave * LPW + ii;                                                   \
            const int p = gi / 16, kind = (gi / 8) & 1;                                       \
            int li = (j_) * KVS + p;                                                          \
            li = li < nact ? li : nact - 1;                                                   \
            const int t = __builtin_amdgcn_readlane(tl.t, li);                                \
            const bool s0 = t < nt0;                                                          \
            const int key0 = s0 ? t * KT : (t - nt0) * KT;                                    \
            const int r = (gi % 8) * 8 + lane / 8;                                            \
            const int lc = swz(r, lane % 8);                                                  \
            const bf16* src;                                                                  \
            if (kind == 0) {                                                                  \
                const int len = s0 ? a.len0 : a.len1;                                         \
                int key = key0 + r;                                                           \
                key = key < len ? key : len - 1;                                              \
                src = (s0 ? K0b : K1b) + (size_t)key * 64 + lc * 8;                           \
            } else {                                                                          \
                src = (s0 ? V0b : V1b) + (size_t)r * (s0 ? a.vstride0 : a.vstride1) + key0 + lc * 8; \
            }                                                                                 \
            load_lds16(src, smem + (sb_) * STAGE_BYTES + (gi / 8) * TILE_BYTES + (gi % 8) * 1024); \
        }                                                                                     \
    } while (0)

    // Q^T fragments (B operand): query q0 + fr, dims 16 ks + 8 fh .. +8.
    bf16x8 qf[4];
    {
        int q = q0 + fr;
        q = q < a.Sq ? q : a.Sq - 1;
        const bf16* qp = a.Q + (bh * a.Sq + q) * 64 + 8 * fh;
#pragma unroll
        for (int ks = 0; ks < 4; ks++) qf[ks] = *reinterpret_cast<const bf16x8*>(qp + 16 * ks);
    }

    f32x16 o[2];
#pragma unroll
    for (int db = 0; db < 2; db++)
#pragma unroll
        for (int e = 0; e < 16; e++) o[db][e] = 0.f;
    float m_run = -INFINITY, l_run = 0.f;

#pragma unroll
    for (int st = 0; st < ST - 1; st++)
        if (st < niter) ATT_ISSUE(st, st);
    for (int j = 0; j < niter; j++) {
        // Stages issued so far: 0 .. min(j + ST - 2, niter - 1); stage j must have landed.
        const int ahead = min(ST - 2, niter - 1 - j);
        if constexpr (ST >= 3) {
            if (ahead >= 1) asm volatile("s_waitcnt vmcnt(%0)" ::"n"(LPW) : "memory");
            else asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        } else {
            (void)ahead;
            asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        }
        raw_barrier();
        if (j + ST - 1 < niter) ATT_ISSUE(j + ST - 1, (j + ST - 1) % ST);
        const int li = j * KVS + par;
        if (li >= nact) continue;  // this parity has no tile in the last iteration
        const unsigned char* kt = smem + (j % ST) * STAGE_BYTES + (2 * par) * TILE_BYTES;
        const unsigned char* vt = kt + TILE_BYTES;

        // S^T for the 64 keys of the tile: two 32-key blocks.
        f32x16 s[2];
#pragma unroll
        for (int kb = 0; kb < 2; kb++) {
#pragma unroll
            for (int e = 0; e < 16; e++) s[kb][e] = 0.f;
#pragma unroll
            for (int ks = 0; ks < 4; ks++)
                s[kb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(frag(kt, 32 * kb + fr, 2 * ks + fh), qf[ks], s[kb], 0, 0, 0);
        }
        // Mask: keys 32 kb + 8 g4 + 4 fh + c of this lane, from the tile's validity bits.
        const unsigned long long vm = ((unsigned long long)(unsigned)__builtin_amdgcn_readlane(tl.hi, li) << 32) |
                                      (unsigned)__builtin_amdgcn_readlane(tl.lo, li);
        if (vm != ~0ull) {
#pragma unroll
            for (int kb = 0; kb < 2; kb++)
#pragma unroll
                for (int g4 = 0; g4 < 4; g4++) {
                    const unsigned nib = (unsigned)(vm >> (32 * kb + 8 * g4 + 4 * fh)) & 15u;
#pragma unroll
                    for (int c = 0; c < 4; c++)
                        if (!((nib >> c) & 1u)) s[kb][4 * g4 + c] = -INFINITY;
                }
        }
        float mx = -INFINITY;
#pragma unroll
        for (int kb = 0; kb < 2; kb++)
#pragma unroll
            for (int e = 0; e < 16; e++) mx = fmaxf(mx, s[kb][e]);
        mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
        const float m_new = fmaxf(m_run, mx);
        const float m_use = m_new == -INFINITY ? 0.f : m_new;
        const float corr = fast_exp2(m_run - m_use);
        float psum = 0.f;
        bf16x8 pf[4];
#pragma unroll
        for (int kb = 0; kb < 2; kb++)
#pragma unroll
            for (int e = 0; e < 16; e++) {
                float p = fast_exp2(s[kb][e] - m_use);
                psum += p;
                pf[2 * kb + (e >> 3)][e & 7] = static_cast<bf16>(p);
            }
        l_run = l_run * corr + psum;
        m_run = m_new;
#pragma unroll
        for (int db = 0; db < 2; db++) o[db] *= corr;
        // O^T += V^T P^T over the 4 16-key groups of the tile.
#pragma unroll
        for (int db = 0; db < 2; db++)
#pragma unroll
            for (int g = 0; g < 4; g++)
                o[db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(frag(vt, 32 * db + fr, 2 * g + fh), pf[g], o[db], 0, 0, 0);
    }
#undef ATT_ISSUE

    // Merge the KVS parities through LDS (reusing the stage buffers; every load has
    // landed since the last iteration waits for all of them): [parity-1][QB][34][64 lanes].
    if constexpr (KVS > 1) {
        __syncthreads();
        float* comb = reinterpret_cast<float*>(smem);
        if (par > 0) {
            float* c = comb + ((size_t)(par - 1) * QB + qb) * 34 * 64 + lane;
#pragma unroll
            for (int db = 0; db < 2; db++)
#pragma unroll
                for (int e = 0; e < 16; e++) c[(16 * db + e) * 64] = o[db][e];
            c[32 * 64] = m_run;
            c[33 * 64] = l_run;
        }
        __syncthreads();
        if (par > 0) return;
#pragma unroll
        for (int pp = 1; pp < KVS; pp++) {
            const float* c = comb + ((size_t)(pp - 1) * QB + qb) * 34 * 64 + lane;
            const float m1 = c[32 * 64], l1 = c[33 * 64];
            const float mt = fmaxf(m_run, m1);
            const float mu = mt == -INFINITY ? 0.f : mt;
            const float c0 = fast_exp2(m_run - mu), c1 = fast_exp2(m1 - mu);
#pragma unroll
            for (int db = 0; db < 2; db++)
#pragma unroll
                for (int e = 0; e < 16; e++) o[db][e] = o[db][e] * c0 + c[(16 * db + e) * 64] * c1;
            l_run = l_run * c0 + l1 * c1;
            m_run = mt;
        }
    }

    // Normalise, gate, store.  o[db][e] = O[q0 + fr][32 db + 8 (e / 4) + 4 fh + e % 4].
    float l = l_run + __shfl_xor(l_run, 32, 64);
    const float inv = l > 0.f ? 1.f / l : 0.f;
    const int q = q0 + fr;
    if (q >= a.Sq) return;
    const size_t m = (size_t)b * a.Sq + q;
#pragma unroll
    for (int db = 0; db < 2; db++)
#pragma unroll
        for (int g4 = 0; g4 < 4; g4++) {
            const int dim = 32 * db + 8 * g4 + 4 * fh;
            if (a.out_mode == 0) {
                const bf16x4 gv = *reinterpret_cast<const bf16x4*>(a.G + m * (a.H * 64) + hh * 64 + dim);
                bf16x4 ov;
#pragma unroll
                for (int c = 0; c < 4; c++) ov[c] = static_cast<bf16>(o[db][4 * g4 + c] * inv * static_cast<float>(gv[c]));
                *reinterpret_cast<bf16x4*>(a.O + m * (a.H * 64) + hh * 64 + dim) = ov;
            } else {
                float* op = a.Of + ((bh * a.Sq) + q) * 64 + dim;
                *reinterpret_cast<float4*>(op) = make_float4(o[db][4 * g4] * inv, o[db][4 * g4 + 1] * inv,
                                                             o[db][4 * g4 + 2] * inv, o[db][4 * g4 + 3] * inv);
            }
        }
}

template <int QB, int KVS, int ST>
int launch_attn32_cfg(const AttnArgs<bf16>& a, hipStream_t st) {
    const size_t lds = (size_t)ST * KVS * 2 * TILE_BYTES;
    static bool attr_set = false;
    if (!attr_set) {
        if (hipFuncSetAttribute((const void*)attn32_kernel<QB, KVS, ST>, hipFuncAttributeMaxDynamicSharedMemorySize,
                                (int)lds) != hipSuccess)
            return -2;
        attr_set = true;
    }
    const int nqb = (a.Sq + 32 * QB - 1) / (32 * QB);
    attn32_kernel<QB, KVS, ST><<<dim3(nqb * a.H * a.B), 64 * QB * KVS, lds, st>>>(a, nqb);
    return 0;
}

}  // namespace

int launch_attention32(const AttnArgs<bf16>& a, hipStream_t st) {
    if (a.Sq <= 0 || a.len0 <= 0 || !a.v_transposed || !a.prescaled || a.mask0) return -1;
    if (a.K1 && !a.bits1) return -1;
    if ((a.vstride0 % KT) || (a.K1 && (a.vstride1 % KT))) return -1;
    const int ntiles = (a.len0 + KT - 1) / KT + (a.K1 ? (a.len1 + KT - 1) / KT : 0);
    if (ntiles > 64) return -1;  // the tile list holds one entry per lane (4096 keys)
    return launch_attn32_cfg<2, 2, 2>(a, st);
}

}  // namespace irodori
