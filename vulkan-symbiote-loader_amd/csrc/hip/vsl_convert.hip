// vsl_convert.hip -- expand GGUF weight storage (F32 / F16 / Q4_0 / Q4_1 / Q8_0) into the packs'
// compute dtype in HBM.
//
// The reference dequantizes on the host inside read_tensor_data (vk_symbiote/src/GGUFLoader.cpp:
// 761-793 -> dequantize_tensor :1121-1223) and uploads the floats.  Here the raw blocks cross PCIe
// (4.5 / 5 / 8.5 bits per weight instead of 32) and one thread expands one 32-element block in HBM.
// Load-time work, HBM-bound: 18-34 bytes in, 64 or 128 bytes out per thread.
//
// Values: every q * d product is exact in binary32 (at most 8 + 11 significant bits, |q * d| >=
// 2^-24 or 0), so the fp32 result does not depend on FMA contraction; fp16 output is that value
// rounded to nearest even.
#include "vsl_device.h"
#include "vsl_internal.h"

namespace {

constexpr int kThreads = 256;

// binary16 -> binary32 by fields.  REF selects the scale helper of dequantize_tensor
// (GGUFLoader.cpp:1132-1149): exponent field 0 gives mantissa * 2^-24 WITHOUT the sign (so -0 -> +0
// and negative subnormals turn positive); everything else is exact binary16.
template <bool REF>
__device__ __forceinline__ float half_bits_to_f32(uint32_t h) {
    const uint32_t s = (h & 0x8000u) << 16, e = (h >> 10) & 31u, m = h & 0x3FFu;
    if (e == 0) {
        const float v = (float)m * 0x1p-24f;  // exact: m < 2^10
        return REF ? v : __uint_as_float(__float_as_uint(v) | s);
    }
    if (e == 31) return __uint_as_float(s | 0x7F800000u | (m << 13));
    return __uint_as_float(s | ((e + 112u) << 23) | (m << 13));
}

template <int FMT>
struct Fmt;
template <> struct Fmt<VSL_WF_Q4_0> { static constexpr int kBytes = 18, kHead = 2; };
template <> struct Fmt<VSL_WF_Q4_1> { static constexpr int kBytes = 20, kHead = 4; };
template <> struct Fmt<VSL_WF_Q8_0> { static constexpr int kBytes = 34, kHead = 2; };

__device__ __forceinline__ void put(float* dst, const float* v) {
#pragma unroll
    for (int j = 0; j < 32; j += 4) *reinterpret_cast<float4v*>(dst + j) = float4v{v[j], v[j + 1], v[j + 2], v[j + 3]};
}
__device__ __forceinline__ void put(vsl_half* dst, const float* v) {
#pragma unroll
    for (int j = 0; j < 32; j += 8) {
        half8 h;
#pragma unroll
        for (int i = 0; i < 8; ++i) h[i] = (vsl_half)v[j + i];
        *reinterpret_cast<half8*>(dst + j) = h;
    }
}

// One thread per 32-element block.
template <int FMT, int LAYOUT, typename OT>
__global__ __launch_bounds__(kThreads) void k_dequant(const uint8_t* __restrict__ src, uint64_t n,
                                                      OT* __restrict__ dst) {
    const uint64_t b = (uint64_t)blockIdx.x * kThreads + threadIdx.x;
    const uint64_t e0 = b * 32;
    if (e0 >= n) return;
    constexpr bool REF = LAYOUT == VSL_QL_REFERENCE;
    // every block starts at an even byte offset (18 / 20 / 34 bytes), so 16-bit loads are aligned
    const uint16_t* p = reinterpret_cast<const uint16_t*>(src + b * Fmt<FMT>::kBytes);
    const float d = half_bits_to_f32<REF>(p[0]);
    const float mn = FMT == VSL_WF_Q4_1 ? half_bits_to_f32<REF>(p[1]) : 0.0f;
    const uint16_t* qs = p + Fmt<FMT>::kHead / 2;
    float v[32];
    if constexpr (FMT == VSL_WF_Q8_0) {
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const uint32_t w = qs[i];
            v[2 * i] = (float)(int8_t)(w & 0xFF) * d;
            v[2 * i + 1] = (float)(int8_t)(w >> 8) * d;
        }
    } else {
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const uint32_t w = qs[i];  // bytes 2i (low half) and 2i+1
#pragma unroll
            for (int k = 0; k < 2; ++k) {
                const int byte = 2 * i + k;
                const uint32_t lo = (w >> (8 * k)) & 15u, hi = (w >> (8 * k + 4)) & 15u;
                // reference: byte -> elements 2*byte, 2*byte+1; ggml: byte -> elements byte, byte+16
                const int e_lo = REF ? 2 * byte : byte, e_hi = REF ? 2 * byte + 1 : byte + 16;
                if constexpr (FMT == VSL_WF_Q4_0) {
                    v[e_lo] = (float)((int)lo - 8) * d;
                    v[e_hi] = (float)((int)hi - 8) * d;
                } else {
                    v[e_lo] = (float)lo * d + mn;
                    v[e_hi] = (float)hi * d + mn;
                }
            }
        }
    }
    if constexpr (sizeof(OT) == 2) {
        // Without this register barrier the backend folds fptrunc(x * d) into v_fma_mix*_f16 with a
        // +0 addend, which turns a -0 product into +0.
#pragma unroll
        for (int j = 0; j < 32; ++j) asm volatile("" : "+v"(v[j]));
    }
    if (e0 + 32 <= n) {
        put(dst + e0, v);
    } else {
#pragma unroll
        for (int j = 0; j < 32; ++j)
            if (e0 + j < n) store_elem(dst + e0 + j, v[j]);
    }
}

// F16 <-> F32 (and same-type copies), elementwise, 32 elements per thread.
template <typename IT, typename OT>
__global__ __launch_bounds__(kThreads) void k_convert_float(const IT* __restrict__ src, uint64_t n,
                                                            OT* __restrict__ dst) {
    const uint64_t e0 = ((uint64_t)blockIdx.x * kThreads + threadIdx.x) * 32;
    if (e0 >= n) return;
#pragma unroll 8
    for (int j = 0; j < 32; ++j)
        if (e0 + j < n) store_elem(dst + e0 + j, to_f32(src[e0 + j]));
}

template <typename OT>
int launch_convert(const void* src, int fmt, int layout, uint64_t n, OT* dst, hipStream_t st) {
    const uint64_t blocks = (n + 32ull * kThreads - 1) / (32ull * kThreads);
    const auto* s8 = static_cast<const uint8_t*>(src);
    const dim3 g((uint32_t)blocks), t(kThreads);
    const bool ref = layout == VSL_QL_REFERENCE;
    switch (fmt) {
        case VSL_WF_F32: k_convert_float<<<g, t, 0, st>>>(static_cast<const float*>(src), n, dst); break;
        case VSL_WF_F16: k_convert_float<<<g, t, 0, st>>>(static_cast<const vsl_half*>(src), n, dst); break;
        case VSL_WF_Q4_0:
            if (ref) k_dequant<VSL_WF_Q4_0, VSL_QL_REFERENCE><<<g, t, 0, st>>>(s8, n, dst);
            else k_dequant<VSL_WF_Q4_0, VSL_QL_GGML><<<g, t, 0, st>>>(s8, n, dst);
            break;
        case VSL_WF_Q4_1:
            if (ref) k_dequant<VSL_WF_Q4_1, VSL_QL_REFERENCE><<<g, t, 0, st>>>(s8, n, dst);
            else k_dequant<VSL_WF_Q4_1, VSL_QL_GGML><<<g, t, 0, st>>>(s8, n, dst);
            break;
        default:
            if (ref) k_dequant<VSL_WF_Q8_0, VSL_QL_REFERENCE><<<g, t, 0, st>>>(s8, n, dst);
            else k_dequant<VSL_WF_Q8_0, VSL_QL_GGML><<<g, t, 0, st>>>(s8, n, dst);
            break;
    }
    HIP_TRY(hipGetLastError());
    return VSL_OK;
}

}  // namespace

extern "C" uint64_t vsl_weight_bytes(int fmt, uint64_t n) {
    switch (fmt) {
        case VSL_WF_F32: return n * 4;
        case VSL_WF_F16: return n * 2;
        case VSL_WF_Q4_0: return (n + 31) / 32 * 18;
        case VSL_WF_Q4_1: return (n + 31) / 32 * 20;
        case VSL_WF_Q8_0: return (n + 31) / 32 * 34;
        default: return 0;
    }
}

extern "C" int vsl_convert_weights(const void* src, int src_fmt, int layout, uint64_t n, void* dst, int dst_dtype,
                                   void* stream) {
    if (src_fmt < VSL_WF_F32 || src_fmt > VSL_WF_Q8_0)
        return vsl_unsupported("vsl_convert_weights: unknown source format %d", src_fmt);
    if (layout != VSL_QL_REFERENCE && layout != VSL_QL_GGML)
        return vsl_invalid("vsl_convert_weights: unknown block layout %d", layout);
    if (dst_dtype != VSL_DT_F32 && dst_dtype != VSL_DT_F16)
        return vsl_unsupported("vsl_convert_weights: output dtype must be F32 or F16");
    if (n == 0) return VSL_OK;
    if (!src || !dst) return vsl_invalid("vsl_convert_weights: null pointer");
    const uintptr_t sa = reinterpret_cast<uintptr_t>(src), da = reinterpret_cast<uintptr_t>(dst);
    if ((sa & (src_fmt == VSL_WF_F32 ? 3 : 1)) || (da & 15))
        return vsl_invalid("vsl_convert_weights: src must be %d-byte and dst 16-byte aligned",
                           src_fmt == VSL_WF_F32 ? 4 : 2);
    const uint64_t sb = vsl_weight_bytes(src_fmt, n), db = n * (dst_dtype == VSL_DT_F16 ? 2 : 4);
    if (sa < da + db && da < sa + sb) return vsl_invalid("vsl_convert_weights: src and dst overlap");
    if ((n + 32ull * kThreads - 1) / (32ull * kThreads) > 0x7FFFFFFFull)
        return vsl_invalid("vsl_convert_weights: n too large");
    hipStream_t st = static_cast<hipStream_t>(stream);
    if (dst_dtype == VSL_DT_F16) return launch_convert(src, src_fmt, layout, n, static_cast<vsl_half*>(dst), st);
    return launch_convert(src, src_fmt, layout, n, static_cast<float*>(dst), st);
}
