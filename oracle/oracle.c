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
