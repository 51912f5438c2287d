// vsl_internal.h -- host-side helpers shared by the C ABI translation units (not installed).
#pragma once
#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdint>

#include "vsl_hip.h"

void vsl_set_error(const char* fmt, ...);
int vsl_hip_fail(hipError_t e, const char* what, const char* file, int line);
uint64_t vsl_derive_key(uint64_t seed, const char* name);

#define HIP_TRY(expr)                                                      \
    do {                                                                   \
        hipError_t _e = (expr);                                            \
        if (_e != hipSuccess) return vsl_hip_fail(_e, #expr, __FILE__, __LINE__); \
    } while (0)

template <typename... A>
static inline int vsl_invalid(const char* fmt, A... a) {
    vsl_set_error(fmt, a...);
    return VSL_E_INVALID;
}
template <typename... A>
static inline int vsl_unsupported(const char* fmt, A... a) {
    vsl_set_error(fmt, a...);
    return VSL_E_UNSUPPORTED;
}
