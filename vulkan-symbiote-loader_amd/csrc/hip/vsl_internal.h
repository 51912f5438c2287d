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

template <typename... A>
static inline int vsl_capacity(const char* fmt, A... a) {
    vsl_set_error(fmt, a...);
    return VSL_E_CAPACITY;
}

// Direct-to-LDS prefill GEMM (vsl_gemm_dma.hip). cfg 0: 256 x 256 tiles, cfg 1: 128 x 256.
// A operand forms: one fp16 plane, VSL_DT_F16X2 (hi/lo fp16 planes), VSL_DT_F16F8 (fp16 hi plane and
// fp8 lo plane); SwiGLU output forms: fp16, VSL_DT_F16X2, VSL_DT_F16F8.
enum { kGemmA1 = 0, kGemmAX2 = 1, kGemmAF8 = 2 };
enum { kGemmC1 = 0, kGemmCX2 = 1, kGemmCF8 = 2 };
uint32_t vsl_gemm_dma_tiles(int cfg, uint32_t M, uint32_t N, uint32_t K, int epi);
// b8s: the weight shift of the fp8 lo product (VSL_GEMM_B8_SHIFT), used by the kGemmAF8 form only.
int vsl_gemm_dma_launch(int cfg, void* stream, const void* A, const void* B, uint32_t M, uint32_t N, uint32_t K,
                        void* C, int epi, int am, int cm, int b8s);
// Split-K plan of the direct-to-LDS GEMM (k chunks of the 128 x 256 tiling, fp32 partials in a
// workspace, an ordered reduction applying the epilogue): returns the split (0: none).
uint32_t vsl_gemm_splitk_plan(uint32_t M, uint32_t N, uint32_t K, int epi, uint32_t min_items, uint64_t* ws_bytes);
// The k-chunk partials alone, ws[chunk][M][N] fp32, for a caller that sums them itself.
void vsl_gemm_splitk_partials(uint32_t ksplit, void* stream, const void* A, const void* B, uint32_t M, uint32_t N,
                              uint32_t K, int am, float* ws, int b8s);
int vsl_gemm_splitk_launch(uint32_t ksplit, void* stream, const void* A, const void* B, uint32_t M, uint32_t N,
                           uint32_t K, void* C, int epi, int am, float* ws, int b8s);
