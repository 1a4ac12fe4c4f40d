// Element-wise and small kernels of the DACVAE decoder (codec/decoder.rs, layers.rs,
// bottleneck.rs).  The convolutions themselves run on the matrix-core GEMM
// (launch_gemm_conv); these kernels produce its operands:
//   * activations are channels-last [frames, Cp] (Cp = channels rounded up to 64, the
//     padded channels exactly zero), so a frame is one GEMM row;
//   * a convolution operand carries `halo` zero rows before and after the frames, which
//     are the convolution's zero padding: the implicit im2col of the GEMM never needs a
//     bounds test for the taps.
#include "common.hpp"
#include "kernels.hpp"

namespace irodori {

namespace {

// Snake1d (layers.rs:24-31) in f32: x + sin(a x)^2 / (a + 1e-9).
__device__ __forceinline__ float snake(float v, float a) {
    const float s = sinf(a * v);
    return v + s * s / (a + 1e-9f);
}

template <typename T>
__device__ __forceinline__ void store8(T* p, const float (&v)[8]) {
    if constexpr (sizeof(T) == 2) {
        bf16x8 h;
#pragma unroll
        for (int i = 0; i < 8; i++) h[i] = static_cast<bf16>(v[i]);
        *reinterpret_cast<bf16x8*>(p) = h;
    } else {
        reinterpret_cast<float4*>(p)[0] = make_float4(v[0], v[1], v[2], v[3]);
        reinterpret_cast<float4*>(p)[1] = make_float4(v[4], v[5], v[6], v[7]);
    }
}

template <typename T>
__device__ __forceinline__ void load8(const T* p, float (&v)[8]) {
    if constexpr (sizeof(T) == 2) {
        const bf16x8 h = *reinterpret_cast<const bf16x8*>(p);
#pragma unroll
        for (int i = 0; i < 8; i++) v[i] = static_cast<float>(h[i]);
    } else {
        const float4 a = reinterpret_cast<const float4*>(p)[0], b = reinterpret_cast<const float4*>(p)[1];
        v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
        v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
    }
}

// One thread per 8 channels of an operand row r in [0, L + 2 halo): Snake of frame
// r - halo of x [L, Cp] (alpha [Cp], zero past the real channels), zeros in the halos.
template <typename T>
__global__ __launch_bounds__(256) void snake_rows_kernel(const float* __restrict__ x, const float* __restrict__ alpha,
                                                         int L, int Cp, int halo, T* __restrict__ s) {
    const int c8 = Cp / 8;
    const long idx = (long)blockIdx.x * 256 + threadIdx.x;
    if (idx >= (long)(L + 2 * halo) * c8) return;
    const int r = (int)(idx / c8), c = (int)(idx % c8) * 8;
    float v[8];
    const int t = r - halo;
    if (t >= 0 && t < L) {
        const float4* px = reinterpret_cast<const float4*>(x + (size_t)t * Cp + c);
        const float4 a0 = px[0], a1 = px[1];
        const float4* pa = reinterpret_cast<const float4*>(alpha + c);
        const float4 b0 = pa[0], b1 = pa[1];
        v[0] = snake(a0.x, b0.x); v[1] = snake(a0.y, b0.y); v[2] = snake(a0.z, b0.z); v[3] = snake(a0.w, b0.w);
        v[4] = snake(a1.x, b1.x); v[5] = snake(a1.y, b1.y); v[6] = snake(a1.z, b1.z); v[7] = snake(a1.w, b1.w);
    } else {
#pragma unroll
        for (int i = 0; i < 8; i++) v[i] = 0.f;
    }
    store8<T>(s + (size_t)r * Cp + c, v);
}

// quantizer.out_proj (bottleneck.rs:21-23, a k 1 Conv1d): one thread per 8 output
// channels of an operand row: s[r] = W lat[r - halo] + b over Cl latent channels, zeros in
// the halos.  W [Pp, Cl] and b [Pp] f32, zero past the real channels.
template <typename T>
__global__ __launch_bounds__(256) void codec_in_kernel(const float* __restrict__ lat, int frames, int Cl,
                                                       const float* __restrict__ w, const float* __restrict__ b,
                                                       int Pp, int halo, T* __restrict__ s) {
    const int c8 = Pp / 8;
    const long idx = (long)blockIdx.x * 256 + threadIdx.x;
    if (idx >= (long)(frames + 2 * halo) * c8) return;
    const int r = (int)(idx / c8), o = (int)(idx % c8) * 8;
    const int t = r - halo;
    float v[8];
#pragma unroll
    for (int i = 0; i < 8; i++) v[i] = 0.f;
    if (t >= 0 && t < frames) {
        const float* lr = lat + (size_t)t * Cl;
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const float* wr = w + (size_t)(o + i) * Cl;
            float acc = 0.f;
            for (int c = 0; c < Cl; c++) acc = fmaf(wr[c], lr[c], acc);
            v[i] = acc + b[o + i];
        }
    }
    store8<T>(s + (size_t)r * Pp + o, v);
}

// WmHead (decoder.rs WmHead::forward): Conv1d(Cp -> 1, k 7, pad 3) over the Snake'd
// operand s [L + 2 halo, Cp] (halo >= 3), then tanh.  One thread per frame; the taps
// w [7, Cp] f32 (w[j Cp + c] = weight[0, c, j], zero past the real channels).
template <typename T>
__global__ __launch_bounds__(256) void codec_head_kernel(const T* __restrict__ s, int L, int Cp, int halo,
                                                         const float* __restrict__ w, const float* __restrict__ b,
                                                         float* __restrict__ wav) {
    const int t = blockIdx.x * 256 + threadIdx.x;
    if (t >= L) return;
    float acc = 0.f;
    for (int j = 0; j < 7; j++) {
        const T* row = s + (size_t)(t + j - 3 + halo) * Cp;
        const float* wj = w + j * Cp;
        for (int c = 0; c < Cp; c += 8) {
            float v[8];
            load8<T>(row + c, v);
#pragma unroll
            for (int i = 0; i < 8; i++) acc = fmaf(wj[c + i], v[i], acc);
        }
    }
    wav[t] = tanhf(acc + (b ? b[0] : 0.f));
}

template <typename T>
__global__ __launch_bounds__(256) void cvt_f32_kernel(const float* __restrict__ src, long n, T* __restrict__ dst) {
    const long i = (long)blockIdx.x * 256 + threadIdx.x;
    if (i < n) dst[i] = from_f32<T>(src[i]);
}

inline unsigned blocks_for(long n) { return (unsigned)((n + 255) / 256); }

}  // namespace

template <typename T>
void launch_codec_snake(const float* x, const float* alpha, int L, int Cp, int halo, T* s, hipStream_t st) {
    const long n = (long)(L + 2 * halo) * (Cp / 8);
    if (n > 0) snake_rows_kernel<T><<<blocks_for(n), 256, 0, st>>>(x, alpha, L, Cp, halo, s);
}

template <typename T>
void launch_codec_in(const float* lat, int frames, int Cl, const float* w, const float* b, int Pp, int halo, T* s,
                     hipStream_t st) {
    const long n = (long)(frames + 2 * halo) * (Pp / 8);
    if (n > 0) codec_in_kernel<T><<<blocks_for(n), 256, 0, st>>>(lat, frames, Cl, w, b, Pp, halo, s);
}

template <typename T>
void launch_codec_head(const T* s, int L, int Cp, int halo, const float* w, const float* b, float* wav,
                       hipStream_t st) {
    if (L > 0) codec_head_kernel<T><<<blocks_for(L), 256, 0, st>>>(s, L, Cp, halo, w, b, wav);
}

template <typename T>
void launch_cvt_f32(const float* src, long n, T* dst, hipStream_t st) {
    if (n > 0) cvt_f32_kernel<T><<<blocks_for(n), 256, 0, st>>>(src, n, dst);
}

#define IRO_CODEC_INST(T)                                                                                   \
    template void launch_codec_snake<T>(const float*, const float*, int, int, int, T*, hipStream_t);          \
    template void launch_codec_in<T>(const float*, int, int, const float*, const float*, int, int, T*,       \
                                     hipStream_t);                                                          \
    template void launch_codec_head<T>(const T*, int, int, int, const float*, const float*, float*, hipStream_t); \
    template void launch_cvt_f32<T>(const float*, long, T*, hipStream_t);
IRO_CODEC_INST(bf16)
IRO_CODEC_INST(float)
#undef IRO_CODEC_INST

}  // namespace irodori
