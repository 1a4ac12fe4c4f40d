// Host-side helpers shared by the library's C entry points (context.hip, encoder.hip):
// status propagation, the exception guard of every entry point, launch checks, and the
// RoPE tables.
#pragma once

#include <cmath>
#include <new>
#include <string>
#include <vector>

#include "../../include/irodori_hip.h"
#include "common.hpp"

#define IRO_TRY(expr)                      \
    do {                                   \
        int _rc = (expr);                  \
        if (_rc != IRODORI_OK) return _rc; \
    } while (0)

#define IRO_GUARD_BEGIN try {
#define IRO_GUARD_END                                     \
    }                                                     \
    catch (const std::bad_alloc&) {                       \
        ::irodori::set_last_error("host allocation failed"); \
        return IRODORI_ERR_OOM;                           \
    }                                                     \
    catch (...) {                                         \
        ::irodori::set_last_error("unexpected C++ exception"); \
        return IRODORI_ERR_HIP;                           \
    }

namespace irodori {

// The last asynchronous launch error, as a status code.
inline int check_launch(const char* what) {
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        set_last_error(std::string(what) + ": " + hipGetErrorString(e));
        return IRODORI_ERR_HIP;
    }
    return IRODORI_OK;
}

// rope.rs:24-63 in f32: freq_i = 1 / theta^(2i/Dh), angle = pos * freq_i.
inline void host_rope_tables(int S, int Dh, float theta, std::vector<float>& cs, std::vector<float>& sn) {
    int half = Dh / 2;
    cs.resize((size_t)S * half);
    sn.resize((size_t)S * half);
    for (int s = 0; s < S; s++)
        for (int i = 0; i < half; i++) {
            float freq = 1.0f / powf(theta, 2.0f * (float)i / (float)Dh);
            float a = (float)s * freq;
            cs[(size_t)s * half + i] = cosf(a);
            sn[(size_t)s * half + i] = sinf(a);
        }
}

}  // namespace irodori
