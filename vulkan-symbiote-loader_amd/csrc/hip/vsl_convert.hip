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
#include <type_traits>

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

// GGUF blocks -> blocks block0 .. of a resident pack (one thread per block): Q8 values as stored,
// Q4 nibbles in the pack's order (value 2j of a block in the low nibble of byte j, 2j + 1 in the high
// one; the reference layout already has it, ggml's holds values j and j + 16 in byte j), the scale
// (and the Q4_1 offset) as the fp32 value k_dequant multiplies by.
template <int FMT, int LAYOUT>
__global__ __launch_bounds__(kThreads) void k_quant_pack(const uint8_t* __restrict__ src, uint64_t n_blocks,
                                                         uint8_t* __restrict__ vals, float* __restrict__ scales,
                                                         float* __restrict__ mins, uint64_t block0) {
    const uint64_t b = (uint64_t)blockIdx.x * kThreads + threadIdx.x;
    if (b >= n_blocks) return;
    constexpr bool REF = LAYOUT == VSL_QL_REFERENCE;
    const uint16_t* p = reinterpret_cast<const uint16_t*>(src + b * Fmt<FMT>::kBytes);
    const uint64_t ob = block0 + b;
    scales[ob] = half_bits_to_f32<REF>(p[0]);
    if constexpr (FMT == VSL_WF_Q4_1) mins[ob] = half_bits_to_f32<REF>(p[1]);
    const uint16_t* qs = p + Fmt<FMT>::kHead / 2;
    if constexpr (FMT == VSL_WF_Q8_0) {
        uint32_t w[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) w[i] = (uint32_t)qs[2 * i] | ((uint32_t)qs[2 * i + 1] << 16);
        uint4* o = reinterpret_cast<uint4*>(vals + ob * 32);
        o[0] = make_uint4(w[0], w[1], w[2], w[3]);
        o[1] = make_uint4(w[4], w[5], w[6], w[7]);
    } else {
        uint8_t in[16], out[16];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            in[2 * i] = (uint8_t)(qs[i] & 0xFF);
            in[2 * i + 1] = (uint8_t)(qs[i] >> 8);
        }
#pragma unroll
        for (int j = 0; j < 16; ++j) {
            if constexpr (REF) {
                out[j] = in[j];
            } else {
                // values 2j and 2j + 1 of the block: ggml keeps value i < 16 in the low nibble of byte i
                // and value i >= 16 in the high nibble of byte i - 16
                auto val = [&](int i) { return i < 16 ? (in[i] & 15u) : (in[i - 16] >> 4); };
                out[j] = (uint8_t)(val(2 * j) | (val(2 * j + 1) << 4));
            }
        }
        uint32_t w[4];
#pragma unroll
        for (int i = 0; i < 4; ++i)
            w[i] = (uint32_t)out[4 * i] | ((uint32_t)out[4 * i + 1] << 8) | ((uint32_t)out[4 * i + 2] << 16) |
                   ((uint32_t)out[4 * i + 3] << 24);
        *reinterpret_cast<uint4*>(vals + ob * 16) = make_uint4(w[0], w[1], w[2], w[3]);
    }
}

// fp16 / fp32 weights -> a resident pack, round to nearest per 32-value block: Q8_0 d = max|w| / 127,
// q = round(w / d); Q4_0 d = -w_max / 8 (w_max the value of largest magnitude), q = clamp(round(w / d)
// + 8, 0, 15); Q4_1 d = (max - min) / 15, m = min, q = clamp(round((w - m) / d), 0, 15).
template <int DT, typename IT>
__global__ __launch_bounds__(kThreads) void k_quantize_pack(const IT* __restrict__ w, uint64_t n_blocks,
                                                            uint8_t* __restrict__ vals, float* __restrict__ scales,
                                                            float* __restrict__ mins) {
    const uint64_t b = (uint64_t)blockIdx.x * kThreads + threadIdx.x;
    if (b >= n_blocks) return;
    float v[32];
#pragma unroll
    for (int i = 0; i < 32; ++i) v[i] = to_f32(w[b * 32 + i]);
    if constexpr (DT == VSL_DT_Q8_0) {
        float amax = 0.f;
#pragma unroll
        for (int i = 0; i < 32; ++i) amax = fmaxf(amax, fabsf(v[i]));
        const float d = amax / 127.f, id = d > 0.f ? 1.f / d : 0.f;
        uint32_t o[8] = {0, 0, 0, 0, 0, 0, 0, 0};
#pragma unroll
        for (int i = 0; i < 32; ++i) {
            const int q = (int)rintf(v[i] * id);
            o[i / 4] |= (uint32_t)(uint8_t)(int8_t)(q < -127 ? -127 : q > 127 ? 127 : q) << (8 * (i % 4));
        }
        uint4* out = reinterpret_cast<uint4*>(vals + b * 32);
        out[0] = make_uint4(o[0], o[1], o[2], o[3]);
        out[1] = make_uint4(o[4], o[5], o[6], o[7]);
        scales[b] = d;
    } else {
        float d, m = 0.f;
        if constexpr (DT == VSL_DT_Q4_0) {
            float wmax = 0.f;
#pragma unroll
            for (int i = 0; i < 32; ++i)
                if (fabsf(v[i]) > fabsf(wmax)) wmax = v[i];
            d = -wmax / 8.f;
        } else {
            float lo = v[0], hi = v[0];
#pragma unroll
            for (int i = 1; i < 32; ++i) {
                lo = fminf(lo, v[i]);
                hi = fmaxf(hi, v[i]);
            }
            d = (hi - lo) / 15.f;
            m = lo;
        }
        const float id = d != 0.f ? 1.f / d : 0.f;
        uint32_t o[4] = {0, 0, 0, 0};
#pragma unroll
        for (int i = 0; i < 32; ++i) {
            int q = DT == VSL_DT_Q4_0 ? (int)rintf(v[i] * id) + 8 : (int)rintf((v[i] - m) * id);
            q = q < 0 ? 0 : q > 15 ? 15 : q;
            o[i / 8] |= (uint32_t)q << (4 * (i % 8));
        }
        *reinterpret_cast<uint4*>(vals + b * 16) = make_uint4(o[0], o[1], o[2], o[3]);
        scales[b] = d;
        if constexpr (DT == VSL_DT_Q4_1) mins[b] = m;
    }
}

// A resident pack -> fp16 / fp32 weights (q * d, (q - 8) * d or q * d + m in fp32).
template <int DT, typename OT>
__global__ __launch_bounds__(kThreads) void k_dequant_pack(const uint8_t* __restrict__ vals,
                                                           const float* __restrict__ scales,
                                                           const float* __restrict__ mins, uint64_t n_blocks,
                                                           OT* __restrict__ dst) {
    const uint64_t b = (uint64_t)blockIdx.x * kThreads + threadIdx.x;
    if (b >= n_blocks) return;
    const float d = scales[b], m = DT == VSL_DT_Q4_1 ? mins[b] : 0.f;
    float v[32];
    if constexpr (DT == VSL_DT_Q8_0) {
        const uint4* p = reinterpret_cast<const uint4*>(vals + b * 32);
        const uint4 a0 = p[0], a1 = p[1];
        const uint32_t w[8] = {a0.x, a0.y, a0.z, a0.w, a1.x, a1.y, a1.z, a1.w};
#pragma unroll
        for (int i = 0; i < 32; ++i) v[i] = (float)(int8_t)(w[i / 4] >> (8 * (i % 4))) * d;
    } else {
        const uint4 a = *reinterpret_cast<const uint4*>(vals + b * 16);
        const uint32_t w[4] = {a.x, a.y, a.z, a.w};
#pragma unroll
        for (int i = 0; i < 32; ++i) {
            const float q = (float)((w[i / 8] >> (4 * (i % 8))) & 15u);
            v[i] = DT == VSL_DT_Q4_0 ? (q - 8.f) * d : q * d + m;
        }
    }
    if constexpr (sizeof(OT) == 2) {
#pragma unroll
        for (int j = 0; j < 32; ++j) asm volatile("" : "+v"(v[j]));
    }
    put(dst + b * 32, v);
}

int qpack_bits(int dtype) { return dtype == VSL_DT_Q8_0 ? 8 : 4; }

}  // namespace

extern "C" uint64_t vsl_quant_pack_bytes(int dtype, uint32_t rows, uint32_t K) {
    if ((dtype != VSL_DT_Q8_0 && dtype != VSL_DT_Q4_0 && dtype != VSL_DT_Q4_1) || K % 32) return 0;
    const int bits = qpack_bits(dtype);
    const uint64_t plane = qpack_align((uint64_t)rows * (K / 32) * 4);
    return (dtype == VSL_DT_Q4_1 ? qpack_mins_off(bits, rows, K) : qpack_scales_off(bits, rows, K)) + plane;
}

extern "C" int vsl_quant_pack(const void* src, int fmt, int layout, uint64_t n_blocks, void* pack, uint32_t rows,
                              uint32_t K, uint64_t block0, void* stream) {
    if (fmt != VSL_WF_Q8_0 && fmt != VSL_WF_Q4_0 && fmt != VSL_WF_Q4_1)
        return vsl_unsupported("vsl_quant_pack: source format %d is not block-quantized", fmt);
    if (layout != VSL_QL_REFERENCE && layout != VSL_QL_GGML) return vsl_invalid("vsl_quant_pack: block layout %d", layout);
    if (K == 0 || K % 32) return vsl_invalid("vsl_quant_pack: K=%u must be a positive multiple of 32", K);
    if (n_blocks == 0) return VSL_OK;
    if (!src || !pack) return vsl_invalid("vsl_quant_pack: null pointer");
    if ((reinterpret_cast<uintptr_t>(src) & 1) || (reinterpret_cast<uintptr_t>(pack) & 255))
        return vsl_invalid("vsl_quant_pack: src must be 2-byte and pack 256-byte aligned");
    if (block0 + n_blocks > (uint64_t)rows * (K / 32)) return vsl_invalid("vsl_quant_pack: blocks past the pack's rows");
    const int dt = fmt == VSL_WF_Q8_0 ? VSL_DT_Q8_0 : fmt == VSL_WF_Q4_0 ? VSL_DT_Q4_0 : VSL_DT_Q4_1;
    const int bits = qpack_bits(dt);
    uint8_t* base = static_cast<uint8_t*>(pack);
    float* sc = reinterpret_cast<float*>(base + qpack_scales_off(bits, rows, K));
    float* mn = reinterpret_cast<float*>(base + qpack_mins_off(bits, rows, K));
    const auto* s8 = static_cast<const uint8_t*>(src);
    const dim3 g((uint32_t)((n_blocks + kThreads - 1) / kThreads)), t(kThreads);
    hipStream_t st = static_cast<hipStream_t>(stream);
    const bool ref = layout == VSL_QL_REFERENCE;
    switch (fmt) {
        case VSL_WF_Q8_0:
            if (ref) k_quant_pack<VSL_WF_Q8_0, VSL_QL_REFERENCE><<<g, t, 0, st>>>(s8, n_blocks, base, sc, mn, block0);
            else k_quant_pack<VSL_WF_Q8_0, VSL_QL_GGML><<<g, t, 0, st>>>(s8, n_blocks, base, sc, mn, block0);
            break;
        case VSL_WF_Q4_0:
            if (ref) k_quant_pack<VSL_WF_Q4_0, VSL_QL_REFERENCE><<<g, t, 0, st>>>(s8, n_blocks, base, sc, mn, block0);
            else k_quant_pack<VSL_WF_Q4_0, VSL_QL_GGML><<<g, t, 0, st>>>(s8, n_blocks, base, sc, mn, block0);
            break;
        default:
            if (ref) k_quant_pack<VSL_WF_Q4_1, VSL_QL_REFERENCE><<<g, t, 0, st>>>(s8, n_blocks, base, sc, mn, block0);
            else k_quant_pack<VSL_WF_Q4_1, VSL_QL_GGML><<<g, t, 0, st>>>(s8, n_blocks, base, sc, mn, block0);
            break;
    }
    HIP_TRY(hipGetLastError());
    return VSL_OK;
}

extern "C" int vsl_quantize_pack(const void* w, int wdtype, uint32_t rows, uint32_t K, int dtype, void* pack,
                                 void* stream) {
    if (dtype != VSL_DT_Q8_0 && dtype != VSL_DT_Q4_0 && dtype != VSL_DT_Q4_1)
        return vsl_unsupported("vsl_quantize_pack: pack dtype %d", dtype);
    if (wdtype != VSL_DT_F16 && wdtype != VSL_DT_F32) return vsl_unsupported("vsl_quantize_pack: weight dtype %d", wdtype);
    if (K == 0 || K % 32) return vsl_invalid("vsl_quantize_pack: K=%u must be a positive multiple of 32", K);
    if (rows == 0) return VSL_OK;
    if (!w || !pack) return vsl_invalid("vsl_quantize_pack: null pointer");
    if ((reinterpret_cast<uintptr_t>(w) & 3) || (reinterpret_cast<uintptr_t>(pack) & 255))
        return vsl_invalid("vsl_quantize_pack: w must be 4-byte and pack 256-byte aligned");
    const uint64_t nb = (uint64_t)rows * (K / 32);
    const int bits = qpack_bits(dtype);
    uint8_t* base = static_cast<uint8_t*>(pack);
    float* sc = reinterpret_cast<float*>(base + qpack_scales_off(bits, rows, K));
    float* mn = reinterpret_cast<float*>(base + qpack_mins_off(bits, rows, K));
    const dim3 g((uint32_t)((nb + kThreads - 1) / kThreads)), t(kThreads);
    hipStream_t st = static_cast<hipStream_t>(stream);
    auto go = [&](auto dtc, auto* in) {
        k_quantize_pack<decltype(dtc)::value><<<g, t, 0, st>>>(in, nb, base, sc, mn);
    };
    using Q8 = std::integral_constant<int, VSL_DT_Q8_0>;
    using Q4 = std::integral_constant<int, VSL_DT_Q4_0>;
    using Q41 = std::integral_constant<int, VSL_DT_Q4_1>;
    auto by_dt = [&](auto* in) {
        if (dtype == VSL_DT_Q8_0) go(Q8{}, in);
        else if (dtype == VSL_DT_Q4_0) go(Q4{}, in);
        else go(Q41{}, in);
    };
    if (wdtype == VSL_DT_F16) by_dt(static_cast<const vsl_half*>(w));
    else by_dt(static_cast<const float*>(w));
    HIP_TRY(hipGetLastError());
    return VSL_OK;
}

extern "C" int vsl_dequant_pack(const void* pack, int dtype, uint32_t rows, uint32_t K, void* w, int wdtype,
                                void* stream) {
    if (dtype != VSL_DT_Q8_0 && dtype != VSL_DT_Q4_0 && dtype != VSL_DT_Q4_1)
        return vsl_unsupported("vsl_dequant_pack: pack dtype %d", dtype);
    if (wdtype != VSL_DT_F16 && wdtype != VSL_DT_F32) return vsl_unsupported("vsl_dequant_pack: weight dtype %d", wdtype);
    if (K == 0 || K % 32) return vsl_invalid("vsl_dequant_pack: K=%u must be a positive multiple of 32", K);
    if (rows == 0) return VSL_OK;
    if (!w || !pack) return vsl_invalid("vsl_dequant_pack: null pointer");
    if ((reinterpret_cast<uintptr_t>(w) & 15) || (reinterpret_cast<uintptr_t>(pack) & 255))
        return vsl_invalid("vsl_dequant_pack: w must be 16-byte and pack 256-byte aligned");
    const uint64_t nb = (uint64_t)rows * (K / 32);
    const int bits = qpack_bits(dtype);
    const uint8_t* base = static_cast<const uint8_t*>(pack);
    const float* sc = reinterpret_cast<const float*>(base + qpack_scales_off(bits, rows, K));
    const float* mn = reinterpret_cast<const float*>(base + qpack_mins_off(bits, rows, K));
    const dim3 g((uint32_t)((nb + kThreads - 1) / kThreads)), t(kThreads);
    hipStream_t st = static_cast<hipStream_t>(stream);
    auto go = [&](auto dtc, auto* out) {
        k_dequant_pack<decltype(dtc)::value><<<g, t, 0, st>>>(base, sc, mn, nb, out);
    };
    using Q8 = std::integral_constant<int, VSL_DT_Q8_0>;
    using Q4 = std::integral_constant<int, VSL_DT_Q4_0>;
    using Q41 = std::integral_constant<int, VSL_DT_Q4_1>;
    auto by_dt = [&](auto* out) {
        if (dtype == VSL_DT_Q8_0) go(Q8{}, out);
        else if (dtype == VSL_DT_Q4_0) go(Q4{}, out);
        else go(Q41{}, out);
    };
    if (wdtype == VSL_DT_F16) by_dt(static_cast<vsl_half*>(w));
    else by_dt(static_cast<float*>(w));
    HIP_TRY(hipGetLastError());
    return VSL_OK;
}

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
