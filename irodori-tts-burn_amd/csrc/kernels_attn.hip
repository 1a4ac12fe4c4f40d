// Joint flash attention on the matrix cores (attention.rs:328-425 / :619-664 semantics):
//   o[q] = sum_j softmax_j(q . k_j / sqrt(Dh) | valid_j) v_j, keys j drawn from two
//   segments read in place — segment 0 = the latent self keys written by the QKV GEMM,
//   segment 1 = the cached text|speaker context keys of this layer — so no [self|ctx]
//   concatenation is ever materialised.  A fully masked query row yields 0.
//
// Formulation: per 64-key tile the wavefront computes S^T = K Q^T (16x16x32 MFMA, K tile
// from LDS as the A operand, Q held in registers as the B operand).  In the resulting
// accumulator layout lane l holds keys 4*(l/16)+i (+16 per block) of query column l%16,
// so the online-softmax max/sum of a query reduce over only 4 lanes (l, l^16, l^32,
// l^48), and the probabilities P^T are already in B-operand layout for O^T = V^T P^T —
// no LDS round trip for P.  The A operand of that product is V^T with the keys of each
// 32-key group permuted so that a lane's 8 keys are one contiguous 16-byte read.  In the
// model path V is stored that way in HBM (by the QKV epilogue and at context ingest), so
// K and V^T tiles both move HBM -> registers -> LDS as plain 16-byte rows; the operator
// entry point (V given as [key][d]) transposes while staging instead.
// Workgroup = 4 wavefronts x 16*QB queries of one (batch row, head); K/V tiles are double
// buffered in LDS with register prefetch; context tiles with no valid key are skipped.
#include "common.hpp"
#include "kernels.hpp"

namespace irodori {

namespace {

constexpr int KT = 64;  // keys per tile
constexpr float kLog2e = 1.4426950408889634f;

template <typename T>
__device__ __forceinline__ Frag<T> lds_frag8(const T* p);
template <>
__device__ __forceinline__ Frag<bf16> lds_frag8<bf16>(const bf16* p) {
    Frag<bf16> f;
    f.v = *reinterpret_cast<const bf16x8*>(p);
    return f;
}
template <>
__device__ __forceinline__ Frag<f16> lds_frag8<f16>(const f16* p) {
    Frag<f16> f;
    f.v = *reinterpret_cast<const f16x8*>(p);
    return f;
}
template <>
__device__ __forceinline__ Frag<float> lds_frag8<float>(const float* p) {
    Frag<float> f;
    float4 lo = *reinterpret_cast<const float4*>(p);
    float4 hi = *reinterpret_cast<const float4*>(p + 4);
    f.v[0] = lo.x; f.v[1] = lo.y; f.v[2] = lo.z; f.v[3] = lo.w;
    f.v[4] = hi.x; f.v[5] = hi.y; f.v[6] = hi.z; f.v[7] = hi.w;
    return f;
}

template <typename T>
__device__ __forceinline__ T vec_elem(const u32x4& v, int e);
template <>
__device__ __forceinline__ bf16 vec_elem<bf16>(const u32x4& v, int e) {
    unsigned w = v[e >> 1];
    unsigned short u = (e & 1) ? (unsigned short)(w >> 16) : (unsigned short)(w & 0xffff);
    return __builtin_bit_cast(bf16, u);
}
template <>
__device__ __forceinline__ f16 vec_elem<f16>(const u32x4& v, int e) {
    unsigned w = v[e >> 1];
    unsigned short u = (e & 1) ? (unsigned short)(w >> 16) : (unsigned short)(w & 0xffff);
    return __builtin_bit_cast(f16, u);
}
template <>
__device__ __forceinline__ float vec_elem<float>(const u32x4& v, int e) {
    // Copy the element into a scalar first: bit-casting the vector-element lvalue
    // directly reads element 0.
    unsigned w = v[e];
    return __builtin_bit_cast(float, w);
}

// Position of key k (0..63) of a tile inside the transposed V tile.
__device__ __forceinline__ int vperm(int k) {
    int c = k >> 5, kk = k & 31;
    return c * 32 + ((kk & 15) >> 2) * 8 + (kk >> 4) * 4 + (kk & 3);
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

template <typename T, int DH, int QB, bool VT, bool PRESCALED>
__global__ __launch_bounds__(256) void attn_kernel(AttnArgs<T> a) {
    constexpr int VEC = 16 / sizeof(T);
    constexpr int LDK = DH + 16 / sizeof(T);   // K tile row stride
    constexpr int LDV = KT + 16 / sizeof(T);   // V^T tile row stride
    constexpr int LOADS = KT * DH / VEC / 256; // 16-byte chunks per thread per K (or V) tile
    constexpr int DC = DH / 32, DB = DH / 16;
    constexpr int WQ = 16 * QB;
    static_assert(LOADS >= 1, "tile");

    __shared__ __attribute__((aligned(16))) T Ks[2][KT * LDK];
    __shared__ __attribute__((aligned(16))) T Vt[2][DH * LDV];
    __shared__ float Ms[2][KT];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int b = blockIdx.z, h = blockIdx.y;
    const int q0 = blockIdx.x * (4 * WQ) + wave * WQ;
    const int fr = lane & 15, g = lane >> 4;
    const float sl2 = PRESCALED ? 1.0f : a.scale * kLog2e;

    // Q^T fragments (B operand): query q0 + 16*qb + fr, dims 32*dc + 8*g .. +8.
    Frag<T> qf[QB][DC];
    const T* qbase = a.Q + ((size_t)b * a.H + h) * a.Sq * DH;
#pragma unroll
    for (int qb = 0; qb < QB; qb++) {
        int q = q0 + 16 * qb + fr;
        q = q < a.Sq ? q : a.Sq - 1;
#pragma unroll
        for (int dc = 0; dc < DC; dc++) qf[qb][dc] = load_frag<T>(qbase + (size_t)q * DH + dc * 32 + g * 8);
    }

    const int nt0 = (a.len0 + KT - 1) / KT;
    const int nt1 = a.K1 ? (a.len1 + KT - 1) / KT : 0;
    const int ntiles = nt0 + nt1;
    const int* tile_on = a.tile_on1 ? a.tile_on1 + b * ((a.stride1 + KT - 1) / KT) : nullptr;
    const size_t bh = (size_t)b * a.H + h;
    const T* K0b = a.K0 + bh * a.stride0 * DH;
    const T* K1b = a.K1 ? a.K1 + bh * a.stride1 * DH : nullptr;
    // V: [key][d] rows (VT = false) or V^T rows of vstride permuted keys (VT = true).
    const T* V0b = a.V0 + bh * (VT ? (size_t)DH * a.vstride0 : (size_t)a.stride0 * DH);
    const T* V1b = a.V1 ? a.V1 + bh * (VT ? (size_t)DH * a.vstride1 : (size_t)a.stride1 * DH) : nullptr;
    const float* M0b = a.mask0 ? a.mask0 + (size_t)b * a.len0 : nullptr;
    const float* M1b = a.mask1 ? a.mask1 + (size_t)b * a.stride1 : nullptr;
    // K chunk c = tid + 256 i: key c / (DH/VEC), elements (c % (DH/VEC)) * VEC..
    const int ckey = tid / (DH / VEC), ccol = (tid % (DH / VEC)) * VEC;
    constexpr int KEY_STEP = 256 / (DH / VEC);
    // V^T chunk c = tid + 256 i: dim c / (KT/VEC), keys (c % (KT/VEC)) * VEC..
    const int vdim = tid / (KT / VEC), vkey = (tid % (KT / VEC)) * VEC;
    constexpr int DIM_STEP = 256 / (KT / VEC);

    u32x4 rk[LOADS], rv[LOADS];
    float rm = 0.f;
// First active tile index >= t (context tiles without a valid key are skipped).
#define ATTN_NEXT(t)                                                                       \
    do {                                                                                   \
        while ((t) < ntiles && (t) >= nt0 && tile_on && tile_on[(t) - nt0] == 0) (t)++;   \
    } while (0)
#define ATTN_GLOAD(t)                                                                      \
    do {                                                                                   \
        const bool s0 = (t) < nt0;                                                         \
        const int key0 = s0 ? (t) * KT : ((t) - nt0) * KT;                                 \
        const int len = s0 ? a.len0 : a.len1;                                              \
        const T* kb = s0 ? K0b : K1b;                                                      \
        const T* vb = s0 ? V0b : V1b;                                                      \
        const float* mk = s0 ? M0b : M1b;                                                  \
        _Pragma("unroll") for (int i = 0; i < LOADS; i++) {                                \
            int key = key0 + ckey + KEY_STEP * i;                                          \
            key = key < len ? key : len - 1;                                               \
            rk[i] = *reinterpret_cast<const u32x4*>(kb + (size_t)key * DH + ccol);         \
            if constexpr (VT) {                                                            \
                const size_t vs = s0 ? a.vstride0 : a.vstride1;                            \
                rv[i] = *reinterpret_cast<const u32x4*>(                                   \
                    vb + (size_t)(vdim + DIM_STEP * i) * vs + key0 + vkey);                \
            } else {                                                                       \
                rv[i] = *reinterpret_cast<const u32x4*>(vb + (size_t)key * DH + ccol);     \
            }                                                                              \
        }                                                                                  \
        if (tid < KT) {                                                                    \
            int key = key0 + tid;                                                          \
            bool ok = key < len && (mk == nullptr || mk[key] >= 0.5f);                     \
            rm = ok ? 0.f : -INFINITY;                                                     \
        }                                                                                  \
    } while (0)
#define ATTN_LSTORE(buf)                                                                   \
    do {                                                                                   \
        _Pragma("unroll") for (int i = 0; i < LOADS; i++) {                                \
            int key = ckey + KEY_STEP * i;                                                 \
            *reinterpret_cast<u32x4*>(&Ks[buf][key * LDK + ccol]) = rk[i];                 \
            if constexpr (VT) {                                                            \
                *reinterpret_cast<u32x4*>(&Vt[buf][(vdim + DIM_STEP * i) * LDV + vkey]) =  \
                    rv[i];                                                                 \
            } else {                                                                       \
                int pk = vperm(key);                                                       \
                _Pragma("unroll") for (int e = 0; e < VEC; e++)                            \
                    Vt[buf][(ccol + e) * LDV + pk] = vec_elem<T>(rv[i], e);                \
            }                                                                              \
        }                                                                                  \
        if (tid < KT) Ms[buf][tid] = rm;                                                   \
    } while (0)

    f32x4 o[DB][QB];
#pragma unroll
    for (int d = 0; d < DB; d++)
#pragma unroll
        for (int qb = 0; qb < QB; qb++) o[d][qb] = f32x4{0.f, 0.f, 0.f, 0.f};
    float m_run[QB], l_run[QB];
#pragma unroll
    for (int qb = 0; qb < QB; qb++) { m_run[qb] = -INFINITY; l_run[qb] = 0.f; }

    int t = 0;
    ATTN_NEXT(t);
    if (t < ntiles) {
        ATTN_GLOAD(t);
        ATTN_LSTORE(0);
    }
    __syncthreads();
    int buf = 0;
    while (t < ntiles) {
        int tn = t + 1;
        ATTN_NEXT(tn);
        if (tn < ntiles) ATTN_GLOAD(tn);
        const T* ks = Ks[buf];
        const T* vt = Vt[buf];

        // S^T = K Q^T for the 64 keys of this tile.
        f32x4 s[4][QB];
#pragma unroll
        for (int kb = 0; kb < 4; kb++) {
#pragma unroll
            for (int qb = 0; qb < QB; qb++) s[kb][qb] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int dc = 0; dc < DC; dc++) {
                Frag<T> kf = lds_frag8<T>(ks + (kb * 16 + fr) * LDK + dc * 32 + g * 8);
#pragma unroll
                for (int qb = 0; qb < QB; qb++) mma16(s[kb][qb], kf, qf[qb][dc]);
            }
        }
        // Online softmax over this tile (log2 domain), per query column.  Latent self
        // tiles are never masked except past the segment end (last tile only).
        const bool masked = t >= nt0 || (t + 1) * KT > a.len0 || M0b != nullptr;
        float bias[4][4];
        if (masked) {
#pragma unroll
            for (int kb = 0; kb < 4; kb++)
#pragma unroll
                for (int i = 0; i < 4; i++) bias[kb][i] = Ms[buf][kb * 16 + 4 * g + i];
        }
#pragma unroll
        for (int qb = 0; qb < QB; qb++) {
            float mx = -INFINITY;
#pragma unroll
            for (int kb = 0; kb < 4; kb++)
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    float v = PRESCALED ? s[kb][qb][i] : s[kb][qb][i] * sl2;
                    if (masked) v += bias[kb][i];
                    s[kb][qb][i] = v;
                    mx = fmaxf(mx, v);
                }
            mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
            mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
            float m_new = fmaxf(m_run[qb], mx);
            float m_use = m_new == -INFINITY ? 0.f : m_new;
            float corr = fast_exp2(m_run[qb] - m_use);
            float psum = 0.f;
#pragma unroll
            for (int kb = 0; kb < 4; kb++)
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    float p = fast_exp2(s[kb][qb][i] - m_use);
                    s[kb][qb][i] = p;
                    psum += p;
                }
            l_run[qb] = l_run[qb] * corr + psum;
            m_run[qb] = m_new;
#pragma unroll
            for (int d = 0; d < DB; d++) o[d][qb] *= corr;
        }
        // O^T += V^T P^T, 32 keys per MFMA.
#pragma unroll
        for (int c = 0; c < 2; c++) {
            Frag<T> pf[QB];
#pragma unroll
            for (int qb = 0; qb < QB; qb++)
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    pf[qb].v[i] = from_f32<T>(s[2 * c][qb][i]);
                    pf[qb].v[4 + i] = from_f32<T>(s[2 * c + 1][qb][i]);
                }
#pragma unroll
            for (int d = 0; d < DB; d++) {
                Frag<T> vf = lds_frag8<T>(vt + (d * 16 + fr) * LDV + c * 32 + g * 8);
#pragma unroll
                for (int qb = 0; qb < QB; qb++) mma16(o[d][qb], vf, pf[qb]);
            }
        }
        if (tn < ntiles) ATTN_LSTORE(buf ^ 1);
        __syncthreads();
        buf ^= 1;
        t = tn;
    }
#undef ATTN_NEXT
#undef ATTN_GLOAD
#undef ATTN_LSTORE

    // Epilogue: normalise, optional sigmoid-gate multiply, store.
    // o[d][qb][i] = O[q = q0 + 16 qb + fr][dim = 16 d + 4 g + i].
#pragma unroll
    for (int qb = 0; qb < QB; qb++) {
        float l = l_run[qb];
        l += __shfl_xor(l, 16, 64);
        l += __shfl_xor(l, 32, 64);
        float inv = l > 0.f ? 1.f / l : 0.f;
        int q = q0 + 16 * qb + fr;
        if (q >= a.Sq) continue;
        size_t m = (size_t)b * a.Sq + q;
#pragma unroll
        for (int d = 0; d < DB; d++) {
            int dim = 16 * d + 4 * g;
            if (a.out_mode == 0) {
                const T* gp = a.G + m * (a.H * DH) + h * DH + dim;
                T* op = a.O + m * (a.H * DH) + h * DH + dim;
#pragma unroll
                for (int i = 0; i < 4; i++) op[i] = from_f32<T>(o[d][qb][i] * inv * to_f32(gp[i]));
            } else {
                float* op = a.Of + (((size_t)b * a.H + h) * a.Sq + q) * DH + dim;
                *reinterpret_cast<float4*>(op) = make_float4(o[d][qb][0] * inv, o[d][qb][1] * inv,
                                                             o[d][qb][2] * inv, o[d][qb][3] * inv);
            }
        }
    }
}

template <typename T, int DH, bool VT, bool PRE>
int launch_q(const AttnArgs<T>& a, int qb, hipStream_t st) {
    int wq = 16 * qb;
    dim3 grid((a.Sq + 4 * wq - 1) / (4 * wq), a.H, a.B);
    if (qb == 1)
        attn_kernel<T, DH, 1, VT, PRE><<<grid, 256, 0, st>>>(a);
    else
        attn_kernel<T, DH, 2, VT, PRE><<<grid, 256, 0, st>>>(a);
    return 0;
}

}  // namespace

// 32 queries per wavefront (better K/V reuse) when that still gives >= 2 workgroups per
// CU of the 256-CU chip; 16 otherwise.
template <typename T, int DH>
int launch_attention(const AttnArgs<T>& a, hipStream_t st) {
    if (a.Sq <= 0 || a.len0 <= 0) return -1;
    if (a.v_transposed && ((a.vstride0 % KT) || (a.K1 && (a.vstride1 % KT)))) return -1;
    long wgs32 = (long)((a.Sq + 127) / 128) * a.H * a.B;
    int qb = wgs32 >= 512 ? 2 : 1;
    if (a.v_transposed)
        return a.prescaled ? launch_q<T, DH, true, true>(a, qb, st) : launch_q<T, DH, true, false>(a, qb, st);
    return a.prescaled ? launch_q<T, DH, false, true>(a, qb, st) : launch_q<T, DH, false, false>(a, qb, st);
}

template int launch_attention<bf16, 64>(const AttnArgs<bf16>&, hipStream_t);
template int launch_attention<bf16, 128>(const AttnArgs<bf16>&, hipStream_t);
template int launch_attention<f16, 64>(const AttnArgs<f16>&, hipStream_t);
template int launch_attention<f16, 128>(const AttnArgs<f16>&, hipStream_t);
template int launch_attention<float, 64>(const AttnArgs<float>&, hipStream_t);
template int launch_attention<float, 128>(const AttnArgs<float>&, hipStream_t);

}  // namespace irodori
