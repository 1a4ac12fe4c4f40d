// Shared device/host helpers for the gfx950 (CDNA4) kernels of libirodori_hip.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <mutex>
#include <string>
#include <vector>

namespace irodori {

// ---------------------------------------------------------------------------------
// Element types.  bf16 is clang's __bf16 storage type; arithmetic is always f32.
// ---------------------------------------------------------------------------------
typedef __bf16 bf16;
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
// IEEE half: the storage type of the f16-input SDPA operator (f16 operands on the f16
// matrix-core instructions, f32 accumulation and softmax).
typedef _Float16 f16;
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x8 __attribute__((ext_vector_type(8)));
// Raw 16-byte register chunk (native vector type, so arrays of it stay in VGPRs).
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float to_f32(float v) { return v; }
__device__ __forceinline__ float to_f32(bf16 v) { return static_cast<float>(v); }
__device__ __forceinline__ float to_f32(f16 v) { return static_cast<float>(v); }

template <typename T>
__device__ __forceinline__ T from_f32(float v);
template <>
__device__ __forceinline__ float from_f32<float>(float v) { return v; }
template <>
__device__ __forceinline__ bf16 from_f32<bf16>(float v) { return static_cast<bf16>(v); }
template <>
__device__ __forceinline__ f16 from_f32<f16>(float v) { return static_cast<f16>(v); }

// Snake1d (codec/layers.rs:24-31): v + sin(a v)^2 / (a + 1e-9), from the channel's
// constants (a, ar = a / pi, hc = 0.5 / (a + 1e-9)).  For bf16 results (rounded to 8 bits)
// sin^2 y = (1 - cos 2y) / 2 with the hardware cosine, which takes revolutions:
// cos(2 a v) = cos_rev(ar v), reduced to [-1/2, 1/2] first; f32 results use sinf.
template <typename T>
__device__ __forceinline__ float snake_eval(float v, float a, float ar, float hc) {
    if constexpr (sizeof(T) == 2) {
        float r = ar * v;
        r -= rintf(r);
        return fmaf(hc, 1.f - __builtin_amdgcn_cosf(r), v);
    } else {
        (void)ar;
        (void)hc;
        const float s = sinf(a * v);
        return v + s * s / (a + 1e-9f);
    }
}

// ---------------------------------------------------------------------------------
// fp8 (e4m3fn) GEMM operands: a 32-wide block of a row is stored as e4m3 codes of
// x * 2^-e with e the smallest integer such that max |x| <= 448 * 2^e, and the E8M0 byte
// 127 + e.  The codes then never exceed 448, where the hardware converter (round to
// nearest even) is exact.
// ---------------------------------------------------------------------------------
// The block exponent from the bits of amax = (1 + f / 2^23) 2^(E - 127):
// amax <= 448 2^e  <=>  e >= E - 135 when f <= 0.75 * 2^23, else e >= E - 134.
__device__ __forceinline__ int mx_exp(float amax) {
    const unsigned u = __float_as_uint(amax);
    const int E = (int)(u >> 23);
    if (E == 0) return amax > 0.f ? -127 : 0;
    const int e = (u & 0x7fffffu) <= 0x600000u ? E - 135 : E - 134;
    return e < -127 ? -127 : (e > 127 ? 127 : e);
}
// Four values -> four e4m3 bytes (little-endian in the word).
__device__ __forceinline__ unsigned pack_e4m3(float v0, float v1, float v2, float v3) {
    int w = __builtin_amdgcn_cvt_pk_fp8_f32(v0, v1, 0, false);
    w = __builtin_amdgcn_cvt_pk_fp8_f32(v2, v3, w, true);
    return (unsigned)w;
}
// Quantize four consecutive values held by each lane of an aligned group of 8 lanes (one
// 32-wide block): every lane of the group must call it.  Stores the lane's 4 codes at q
// and, from the group's first lane, the block's scale byte at s.
__device__ __forceinline__ void mx_store4_group8(float a, float b, float c, float d, uint8_t* q, uint8_t* s,
                                                 int lane) {
    float amax = fmaxf(fmaxf(fabsf(a), fabsf(b)), fmaxf(fabsf(c), fabsf(d)));
    amax = fmaxf(amax, __shfl_xor(amax, 1));
    amax = fmaxf(amax, __shfl_xor(amax, 2));
    amax = fmaxf(amax, __shfl_xor(amax, 4));
    const int e = mx_exp(amax);
    *reinterpret_cast<unsigned*>(q) = pack_e4m3(ldexpf(a, -e), ldexpf(b, -e), ldexpf(c, -e), ldexpf(d, -e));
    if ((lane & 7) == 0) *s = (uint8_t)(127 + e);
}

// A "k32 fragment": the 8 consecutive reduction-dim elements one lane feeds to the
// matrix core per 32-wide slice of K.  For bf16 that is one v_mfma_f32_16x16x32_bf16
// operand; for f32 it is the operands of eight v_mfma_f32_16x16x4_f32 (element j goes
// to the j-th instruction).  Both operands of a product use the same element order, so
// the k index each element stands for only has to agree between A and B.
template <typename T>
struct Frag;
template <>
struct Frag<bf16> {
    bf16x8 v;
};
template <>
struct Frag<float> {
    f32x8 v;
};
template <>
struct Frag<f16> {
    f16x8 v;
};

__device__ __forceinline__ void mma16(f32x4& acc, const Frag<bf16>& a, const Frag<bf16>& b) {
    acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a.v, b.v, acc, 0, 0, 0);
}
__device__ __forceinline__ void mma16(f32x4& acc, const Frag<f16>& a, const Frag<f16>& b) {
    acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(a.v, b.v, acc, 0, 0, 0);
}
__device__ __forceinline__ void mma16(f32x4& acc, const Frag<float>& a, const Frag<float>& b) {
#pragma unroll
    for (int j = 0; j < 8; j++) acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a.v[j], b.v[j], acc, 0, 0, 0);
}

// 16-byte vector loads/stores.
template <typename V>
__device__ __forceinline__ V ld_vec(const void* p) {
    return *reinterpret_cast<const V*>(p);
}
template <typename V>
__device__ __forceinline__ void st_vec(void* p, const V& v) {
    *reinterpret_cast<V*>(p) = v;
}

// Load a k32 fragment (8 contiguous elements) from LDS or global memory.
template <typename T>
__device__ __forceinline__ Frag<T> load_frag(const T* p);
template <>
__device__ __forceinline__ Frag<bf16> load_frag<bf16>(const bf16* p) {
    Frag<bf16> f;
    f.v = *reinterpret_cast<const bf16x8*>(p);
    return f;
}
template <>
__device__ __forceinline__ Frag<float> load_frag<float>(const float* p) {
    Frag<float> f;
    f.v = *reinterpret_cast<const f32x8*>(p);
    return f;
}
template <>
__device__ __forceinline__ Frag<f16> load_frag<f16>(const f16* p) {
    Frag<f16> f;
    f.v = *reinterpret_cast<const f16x8*>(p);
    return f;
}

// ---------------------------------------------------------------------------------
// Wavefront (64 lanes) reductions.
// ---------------------------------------------------------------------------------
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
    return v;
}

// v_rcp_f32 (1 ulp) instead of an IEEE division: these feed bf16 operands or are far
// inside the f32 tolerance, and the precise divide is ~10 instructions per element.
__device__ __forceinline__ float silu_f(float v) { return v * __builtin_amdgcn_rcpf(1.0f + __expf(-v)); }
__device__ __forceinline__ float sigmoid_f(float v) { return __builtin_amdgcn_rcpf(1.0f + __expf(-v)); }

// (b, s) = divmod(row, S) without an integer division: a float-reciprocal quotient
// (exact to within one for row < 2^24) and a one-step correction.
__device__ __forceinline__ void row_bs(int row, int S, float inv_s, int& b, int& s) {
    int q = (int)((float)row * inv_s);
    int r = row - q * S;
    if (r < 0) { q--; r += S; }
    if (r >= S) { q++; r -= S; }
    b = q;
    s = r;
}

// Map a linear workgroup id so that consecutive ids land on the same XCD.  Workgroups
// are dispatched round-robin over the 8 XCDs (id % 8); when the grid is a multiple of
// 8 this returns an id such that XCD x owns the contiguous range [x*n/8, (x+1)*n/8).
__device__ __forceinline__ int xcd_remap(int id, int n) {
    if (n % 8) return id;
    return (id % 8) * (n / 8) + id / 8;
}

// ---------------------------------------------------------------------------------
// Host-side error plumbing (thread-local last error, status codes of irodori_hip.h).
// ---------------------------------------------------------------------------------
void set_last_error(const std::string& msg);

// Device allocation of one object's persistent buffers (a DiT context, an encoder, a codec):
// hipMalloc, the pointer recorded in allocs (freed with the object), the bytes added to total.
// With IRODORI_DEVICE_ALLOC_LIMIT set (a byte count, read at each call), an allocation that
// would bring the object's total above it fails with IRODORI_ERR_OOM before hipMalloc runs,
// so a caller can exercise its out-of-memory handling on any device.
int tracked_alloc(std::vector<void*>& allocs, uint64_t& total, void** p, size_t bytes);

// Raises a kernel's dynamic-LDS limit once per process and device (the attribute belongs to
// the kernel's code object on each device; launches run on the current device, which every
// entry point sets to its object's).  The first launch of a kernel variant may come from
// several host threads at once (one context, encoder or codec per thread), so the one-time
// call is guarded by a once_flag per device, owned by the caller (one static LdsLimit per
// kernel instantiation); every caller sees the call's result.
struct LdsLimit {
    static constexpr int kDevices = 64;
    std::once_flag once[kDevices];
    hipError_t rc[kDevices] = {};
};
inline hipError_t set_lds_limit_once(LdsLimit& lim, const void* fn, int bytes) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    if (dev < 0 || dev >= LdsLimit::kDevices) return hipErrorInvalidDevice;
    std::call_once(lim.once[dev],
                   [&] { lim.rc[dev] = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, bytes); });
    return lim.rc[dev];
}

}  // namespace irodori

#define IRO_HIP_CHECK(expr)                                                                 \
    do {                                                                                    \
        hipError_t _e = (expr);                                                             \
        if (_e != hipSuccess) {                                                             \
            ::irodori::set_last_error(std::string(#expr) + ": " + hipGetErrorString(_e));   \
            return _e == hipErrorOutOfMemory ? IRODORI_ERR_OOM : IRODORI_ERR_HIP;          \
        }                                                                                   \
    } while (0)

#define IRO_REQUIRE(cond, code, msg)                                                        \
    do {                                                                                    \
        if (!(cond)) {                                                                      \
            ::irodori::set_last_error(msg);                                                 \
            return code;                                                                    \
        }                                                                                   \
    } while (0)
