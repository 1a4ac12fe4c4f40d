// The SDPA operator entry points (native_fa_sdpa_wgsl / native_fa_sdpa_f16_in,
// fused_sdpa_native.rs:220-302, fused_sdpa_native_f16.rs:181-200): argument checks, the
// choice between the model's joint attention kernel (16-bit operands, head_dim 64, after
// staging Q / V^T / key bits) and the generic flash kernel, and the staging buffer --
// stream-ordered per call (irodori_op_sdpa) or a fixed per-GPU device array
// (irodori_op_sdpa_noalloc, for callers that cannot allocate).
#include <atomic>
#include <mutex>

#include "../../include/irodori_hip.h"
#include "common.hpp"
#include "host.hpp"
#include "kernels.hpp"

using namespace irodori;

namespace {

int check_sdpa_args(int dtype, const void* q, const void* k, const void* v, int B, int H, int Sq, int Skv, int Dh,
                    const float* out) {
    IRO_REQUIRE(q && k && v && out, IRODORI_ERR_INVALID_ARG, "null argument");
    IRO_REQUIRE(B > 0 && H > 0 && Sq > 0 && Skv > 0, IRODORI_ERR_SHAPE, "SDPA dims must be positive");
    IRO_REQUIRE(Dh == 64 || Dh == 128, IRODORI_ERR_SHAPE, "head_dim must be 64 or 128");
    IRO_REQUIRE(dtype == IRODORI_DTYPE_F32 || dtype == IRODORI_DTYPE_BF16 || dtype == IRODORI_DTYPE_F16,
                IRODORI_ERR_DTYPE, "dtype must be F32, BF16 or F16");
    return IRODORI_OK;
}

// 16-bit operands with Dh = 64 run on the model's joint attention kernel after staging
// (its tile list holds up to 16384 keys); everything else on the generic flash kernel.
bool sdpa_staged(int dtype, int Dh, int Skv) {
    return dtype != IRODORI_DTYPE_F32 && Dh == 64 && Skv <= 64 * kAttnMaxKeyTiles;
}

template <typename T>
int sdpa_direct_t(const void* q, const void* k, const void* v, const float* mask, int B, int H, int Sq, int Skv, int Dh,
                  float scale, float* out, hipStream_t st) {
    AttnArgs<T> a{};
    a.Q = static_cast<const T*>(q);
    a.K0 = static_cast<const T*>(k);
    a.V0 = static_cast<const T*>(v);
    a.len0 = Skv; a.stride0 = Skv; a.mask0 = mask;
    a.B = B; a.H = H; a.Sq = Sq; a.scale = scale; a.out_mode = 1; a.Of = out;
    const int rc = Dh == 64 ? launch_attention<T, 64>(a, st) : launch_attention<T, 128>(a, st);
    IRO_REQUIRE(rc == 0, IRODORI_ERR_SHAPE, "sdpa launch rejected the shape");
    return check_launch("sdpa");
}

int sdpa_direct(int dtype, const void* q, const void* k, const void* v, const float* mask, int B, int H, int Sq,
                int Skv, int Dh, float scale, float* out, hipStream_t st) {
    if (dtype == IRODORI_DTYPE_BF16) return sdpa_direct_t<bf16>(q, k, v, mask, B, H, Sq, Skv, Dh, scale, out, st);
    if (dtype == IRODORI_DTYPE_F16) return sdpa_direct_t<f16>(q, k, v, mask, B, H, Sq, Skv, Dh, scale, out, st);
    return sdpa_direct_t<float>(q, k, v, mask, B, H, Sq, Skv, Dh, scale, out, st);
}

// The staged path on a caller-provided (or stream-ordered) buffer ws of `bytes`.
int sdpa_run_staged(int dtype, const void* q, const void* k, const void* v, const float* mask, int B, int H, int Sq,
                    int Skv, float scale, float* out, void* ws, size_t bytes, hipStream_t st) {
    int rc;
    if (dtype == IRODORI_DTYPE_BF16)
        rc = launch_sdpa_staged<bf16>(static_cast<const bf16*>(q), static_cast<const bf16*>(k),
                                      static_cast<const bf16*>(v), mask, B, H, Sq, Skv, scale, out, ws, bytes, st);
    else
        rc = launch_sdpa_staged<f16>(static_cast<const f16*>(q), static_cast<const f16*>(k),
                                     static_cast<const f16*>(v), mask, B, H, Sq, Skv, scale, out, ws, bytes, st);
    IRO_REQUIRE(rc == 0, IRODORI_ERR_SHAPE, "staged sdpa rejected the shape");
    return check_launch("sdpa");
}

// ---- fixed staging buffer of irodori_op_sdpa_noalloc ------------------------------------
// One array per GPU the library runs on, held until the process ends.  In host code its
// name is a host-side stand-in: kernels get the device address that hipGetSymbolAddress
// returns for the current device, looked up once per device.
static __device__ __align__(256) unsigned char scratch[IRODORI_SDPA_SCRATCH_BYTES];

constexpr int kMaxDevices = 64;
std::once_flag g_scratch_once[kMaxDevices];
std::atomic<void*> g_scratch_ptr[kMaxDevices] = {};
hipError_t g_scratch_rc[kMaxDevices] = {};

// The scratch address on the device of `st`, which must be the current device (the address
// is looked up with that device current, and the kernels run on the stream's device), or a
// status code.  The lookup happens on the first call on a device; it is refused while `st`
// is capturing (a first call inside a graph capture), so capturing callers make one eager
// call first.
int scratch_for_stream(hipStream_t st, void** out) {
    int dev = -1;
    IRO_HIP_CHECK(hipGetDevice(&dev));
    if (st) {
        int sdev = -1;
        IRO_HIP_CHECK(hipStreamGetDevice(st, &sdev));
        IRO_REQUIRE(sdev == dev, IRODORI_ERR_INVALID_ARG,
                    "irodori_op_sdpa_noalloc: the stream belongs to device " + std::to_string(sdev) +
                        " but device " + std::to_string(dev) + " is current; make the stream's device current");
    }
    IRO_REQUIRE(dev >= 0 && dev < kMaxDevices, IRODORI_ERR_INVALID_ARG, "device index beyond the scratch table");
    if (!g_scratch_ptr[dev].load()) {
        hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
        IRO_HIP_CHECK(hipStreamIsCapturing(st, &cs));
        IRO_REQUIRE(cs == hipStreamCaptureStatusNone, IRODORI_ERR_INVALID_ARG,
                    "irodori_op_sdpa_noalloc: the first call on a device must not be under graph capture "
                    "(it looks up the fixed buffer's address); make one call outside the capture first");
    }
    std::call_once(g_scratch_once[dev], [dev] {
        void* p = nullptr;
        g_scratch_rc[dev] = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        g_scratch_ptr[dev].store(p);
    });
    void* p = g_scratch_ptr[dev].load();
    if (g_scratch_rc[dev] != hipSuccess || !p) {
        set_last_error(std::string("hipGetSymbolAddress(scratch): ") + hipGetErrorString(g_scratch_rc[dev]));
        return IRODORI_ERR_HIP;
    }
    *out = p;
    return IRODORI_OK;
}

}  // namespace

extern "C" {

int irodori_op_sdpa(int dtype, const void* q, const void* k, const void* v, const float* mask, int B, int H, int Sq,
                    int Skv, int Dh, float scale, float* out, void* stream) {
    IRO_GUARD_BEGIN
    IRO_TRY(check_sdpa_args(dtype, q, k, v, B, H, Sq, Skv, Dh, out));
    hipStream_t st = static_cast<hipStream_t>(stream);
    if (!sdpa_staged(dtype, Dh, Skv)) return sdpa_direct(dtype, q, k, v, mask, B, H, Sq, Skv, Dh, scale, out, st);
    // Staging buffer in stream order: overlapping calls on different streams never share it.
    const size_t bytes = sdpa_stage_bytes(B, H, Sq, Skv);
    void* ws = nullptr;
    IRO_HIP_CHECK(hipMallocAsync(&ws, bytes, st));
    const int rc = sdpa_run_staged(dtype, q, k, v, mask, B, H, Sq, Skv, scale, out, ws, bytes, st);
    const hipError_t fe = hipFreeAsync(ws, st);
    if (rc != IRODORI_OK) return rc;
    IRO_HIP_CHECK(fe);
    return IRODORI_OK;
    IRO_GUARD_END
}

int irodori_op_sdpa_noalloc(int dtype, const void* q, const void* k, const void* v, const float* mask, int B, int H,
                            int Sq, int Skv, int Dh, float scale, float* out, void* stream) {
    IRO_GUARD_BEGIN
    IRO_TRY(check_sdpa_args(dtype, q, k, v, B, H, Sq, Skv, Dh, out));
    hipStream_t st = static_cast<hipStream_t>(stream);
    if (!sdpa_staged(dtype, Dh, Skv)) return sdpa_direct(dtype, q, k, v, mask, B, H, Sq, Skv, Dh, scale, out, st);
    const size_t bytes = sdpa_stage_bytes(B, H, Sq, Skv);
    IRO_REQUIRE(bytes <= IRODORI_SDPA_SCRATCH_BYTES, IRODORI_ERR_SHAPE,
                "irodori_op_sdpa_noalloc: the staging of this shape takes " + std::to_string(bytes) +
                    " bytes, above the fixed " + std::to_string((size_t)IRODORI_SDPA_SCRATCH_BYTES) +
                    "-byte buffer; use irodori_op_sdpa");
    void* ws = nullptr;
    IRO_TRY(scratch_for_stream(st, &ws));
    // The staging kernel writes every byte the attention kernel reads (Q rows, V^T with zero
    // keys past seq_kv, the key bits), so nothing left by an earlier call is read.
    return sdpa_run_staged(dtype, q, k, v, mask, B, H, Sq, Skv, scale, out, ws, IRODORI_SDPA_SCRATCH_BYTES, st);
    IRO_GUARD_END
}

}  // extern "C"
