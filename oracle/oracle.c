/*
 * CPU oracle — TEST INFRASTRUCTURE ONLY (see oracle.h).  Instantiates oracle_body.h
 * in float (orc_f32_*) and double (orc_f64_*) arithmetic.
 */
#include "oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

void orc_set_threads(int n) {
#ifdef _OPENMP
    if (n > 0) omp_set_num_threads(n);
#else
    (void)n;
#endif
}

int orc_get_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}

/* ---- fp8 (e4m3fn) GEMM operands ----
 * The HIP path's fp8 compute mode has no counterpart in the reference (whose backends run
 * f32 / f16 / bf16); these functions define the quantized arithmetic it implements:
 *   weights: per output channel n, s_n = max_k |w[k,n]| / 448 (f32), q = e4m3(w / s_n);
 *   GEMM activations (the A operand): per row and block of 32 consecutive k, a power of
 *   two 2^e with e the smallest integer such that amax <= 448 * 2^e (no saturation),
 *   q = e4m3(x * 2^-e), the scale stored as the E8M0 byte 127 + e;
 *   y[m,n] = s_n * sum_k (q_a 2^e)[m,k] * q_w[k,n].
 * e4m3fn: 1 sign, 4 exponent (bias 7), 3 mantissa bits; max 448; 0x7F / 0xFF are NaN;
 * subnormals are multiples of 2^-9.  Rounding is to nearest, ties to even. */
uint8_t orc_e4m3_encode(float x) {
    uint32_t u;
    memcpy(&u, &x, 4);
    const uint8_t sign = (uint8_t)((u >> 24) & 0x80);
    const float a = fabsf(x);
    if (!(a <= 448.f)) return sign | 0x7E; /* saturate (never reached by the scaled operands) */
    if (a < 0.015625f) {                   /* below 2^-6: the subnormal grid 2^-9 */
        const float q = nearbyintf(a * 512.f); /* default rounding mode: ties to even */
        return sign | (uint8_t)q;          /* q = 8 is 2^-6, code 0x08 */
    }
    memcpy(&u, &a, 4);
    u += 0x7FFFFu + ((u >> 20) & 1u);      /* round the f32 mantissa to 3 bits, ties to even */
    const int e = (int)(u >> 23) - 127;
    return sign | (uint8_t)(((e + 7) << 3) | ((u >> 20) & 7u));
}

float orc_e4m3_decode(uint8_t b) {
    const int e = (b >> 3) & 15, m = b & 7;
    float v;
    if ((b & 0x7F) == 0x7F) v = NAN;
    else if (e == 0) v = ldexpf((float)m, -9);
    else v = ldexpf(1.f + (float)m / 8.f, e - 7);
    return (b & 0x80) ? -v : v;
}

int orc_mx_scale_exp(float amax) {
    if (!(amax > 0.f)) return 0;
    int p;
    const float m = frexpf(amax, &p); /* amax = m 2^p, m in [0.5, 1); 448 = 0.875 2^9 */
    int e = m <= 0.875f ? p - 9 : p - 8;
    return e < -127 ? -127 : (e > 127 ? 127 : e);
}

void orc_mx_quantize_rows(const float* x, int M, int K, uint8_t* q, uint8_t* s) {
    const int nb = K / 32;
    for (int i = 0; i < M; i++)
        for (int blk = 0; blk < nb; blk++) {
            const float* xb = x + (size_t)i * K + 32 * blk;
            float amax = 0.f;
            for (int j = 0; j < 32; j++) amax = fmaxf(amax, fabsf(xb[j]));
            const int e = orc_mx_scale_exp(amax);
            s[(size_t)i * nb + blk] = (uint8_t)(127 + e);
            for (int j = 0; j < 32; j++) q[(size_t)i * K + 32 * blk + j] = orc_e4m3_encode(ldexpf(xb[j], -e));
        }
}

void orc_mx_dequantize_rows(const uint8_t* q, const uint8_t* s, int M, int K, float* y) {
    const int nb = K / 32;
    for (int i = 0; i < M; i++)
        for (int k = 0; k < K; k++)
            y[(size_t)i * K + k] = ldexpf(orc_e4m3_decode(q[(size_t)i * K + k]), (int)s[(size_t)i * nb + k / 32] - 127);
}

void orc_quant_weight_cols(const float* w, int K, int N, uint8_t* q, float* scale) {
    for (int n = 0; n < N; n++) {
        float amax = 0.f;
        for (int k = 0; k < K; k++) amax = fmaxf(amax, fabsf(w[(size_t)k * N + n]));
        const float sn = amax > 0.f ? amax / 448.f : 1.f;
        scale[n] = sn;
        for (int k = 0; k < K; k++) q[(size_t)k * N + n] = orc_e4m3_encode(w[(size_t)k * N + n] / sn);
    }
}

/* ---- float instantiation ---- */
#define R float
#define R_C(v) ((float)(v))
#define P(name) orc_f32_##name
#define LOG logf
#define EXP expf
#define COS cosf
#define SIN sinf
#define POW powf
#define SQRT sqrtf
#define TANH tanhf
#include "oracle_body.h"
#undef R
#undef R_C
#undef P
#undef LOG
#undef EXP
#undef COS
#undef SIN
#undef POW
#undef SQRT
#undef TANH
#undef ORC_IB
#undef ORC_JB

/* ---- double instantiation ---- */
#define R double
#define R_C(v) ((double)(v))
#define P(name) orc_f64_##name
#define LOG log
#define EXP exp
#define COS cos
#define SIN sin
#define POW pow
#define SQRT sqrt
#define TANH tanh
#include "oracle_body.h"
