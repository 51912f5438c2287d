// vsl_device.h -- device-side helpers shared by the gfx950 kernels (wave64, CDNA4).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#define VSL_WAVE 64

typedef _Float16 vsl_half;
typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half2v __attribute__((ext_vector_type(2)));
typedef _Float16 half4 __attribute__((ext_vector_type(4)));
typedef float float4v __attribute__((ext_vector_type(4)));
typedef float float16v __attribute__((ext_vector_type(16)));

// Weight / cache element types used as template parameters. kBits: bits per stored weight value;
// kQuant: a resident block-quantized pack (values plane, then one fp32 scale per 32 values, for WQ41
// also one fp32 offset per 32 values; see vsl_hip.h, VSL_DT_Q8_0 .. VSL_DT_Q4_1).
struct WF16 { typedef vsl_half T; static constexpr int kVec = 8, kBits = 16; static constexpr bool kQuant = false, kMin = false; };
struct WF32 { typedef float T; static constexpr int kVec = 4, kBits = 32; static constexpr bool kQuant = false, kMin = false; };
struct WQ8 { typedef int8_t T; static constexpr int kVec = 16, kBits = 8; static constexpr bool kQuant = true, kMin = false; };
struct WQ4 { typedef uint8_t T; static constexpr int kVec = 32, kBits = 4; static constexpr bool kQuant = true, kMin = false; };
struct WQ41 { typedef uint8_t T; static constexpr int kVec = 32, kBits = 4; static constexpr bool kQuant = true, kMin = true; };

// Byte offset of element e of a row-major weight matrix.
template <class WT>
__device__ __host__ __forceinline__ constexpr uint64_t wt_bytes(uint64_t e) {
    return WT::kBits >= 8 ? e * (WT::kBits / 8) : e / (8 / WT::kBits);
}

// Planes of a block-quantized pack of `rows` x K values (K % 32 == 0): the values, then the fp32
// scales (one per 32 values, row-major block order), then for Q4_1 the fp32 offsets; each plane
// starts at a multiple of 256 bytes.
__device__ __host__ __forceinline__ constexpr uint64_t qpack_align(uint64_t b) { return (b + 255) & ~(uint64_t)255; }
__device__ __host__ __forceinline__ constexpr uint64_t qpack_scales_off(int bits, uint64_t rows, uint64_t K) {
    return qpack_align(rows * K * (uint64_t)bits / 8);
}
__device__ __host__ __forceinline__ constexpr uint64_t qpack_mins_off(int bits, uint64_t rows, uint64_t K) {
    return qpack_scales_off(bits, rows, K) + qpack_align(rows * (K / 32) * 4);
}

__device__ __forceinline__ float to_f32(vsl_half h) { return (float)h; }
__device__ __forceinline__ float to_f32(float f) { return f; }
__device__ __forceinline__ void store_elem(vsl_half* p, float v) { *p = (vsl_half)v; }
__device__ __forceinline__ void store_elem(float* p, float v) { *p = v; }

// 16-byte global load, returned as 4 dwords.  nt=true marks the access streaming (non-temporal),
// used for weights that are read exactly once per token.
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

template <bool NT>
__device__ __forceinline__ uint4 load16(const void* p) {
    u32x4 v;
    if constexpr (NT)
        v = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
    else
        v = *reinterpret_cast<const u32x4*>(p);
    return make_uint4(v.x, v.y, v.z, v.w);
}

// 16 bytes per lane from global memory straight into LDS: lane i writes lds + 16 i (lds is
// wave-uniform). Only the device pass sees the builtin: in the host pass it would invalidate the
// kernel and drop its launch stub.
// The source is a wave-uniform base plus a 32-bit per-lane byte offset (the saddr + voffset form,
// one VGPR per load).
__device__ __forceinline__ void lds_load16(const vsl_half* base, uint32_t byte_off, vsl_half* lds) {
#if defined(__HIP_DEVICE_COMPILE__)
    __builtin_amdgcn_global_load_lds(reinterpret_cast<const char*>(base) + byte_off, lds, 16, 0, 0);
#else
    (void)base;
    (void)byte_off;
    (void)lds;
#endif
}

// LDS transpose read (ds_read_b64_tr_b16): within each group of 16 lanes, lane i receives as its
// value j element i%4 of the four 16-bit values at the address given by lane 4j + i/4 of the group
// (layout measured on gfx950). p must point into LDS, 8-byte aligned.
__device__ __forceinline__ half4 lds_read_tr16(const vsl_half* p) {
    typedef short s4 __attribute__((ext_vector_type(4)));
    const s4 v = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) s4*)(p));
    return __builtin_bit_cast(half4, v);
}

// s_waitcnt vmcnt(n) (gfx9 encoding: vmcnt bits [3:0] and [15:14]; expcnt and lgkmcnt not waited)
#define VSL_VMCNT_WAIT(n) __builtin_amdgcn_s_waitcnt(((n) & 15) | (7 << 4) | (15 << 8) | (((n) >> 4) << 14))
// s_waitcnt lgkmcnt(0) (vmcnt and expcnt not waited)
#define VSL_LGKM_WAIT0() __builtin_amdgcn_s_waitcnt(15 | (7 << 4) | (0 << 8) | (3 << 14))

// hi/lo split of an fp32 value into two binary16 values (hi + lo carries ~22 significant bits).
// hi passes through an empty register asm: stored and subtracted, it is then the same rounded value
// (the backend otherwise may pack the stored hi with a second conversion of v whose rounding need
// not match the one lo was derived from, measured as one fp16 ulp of error in vector stores).
__device__ __forceinline__ void split_f16(float v, vsl_half& hi, vsl_half& lo) {
    hi = (vsl_half)v;
    asm volatile("" : "+v"(hi));
    lo = (vsl_half)(v - (float)hi);
}

// hi / lo8 split of an fp32 value (VSL_DT_F16F8): hi = fp16(v) as in split_f16, and the remainder
// v - hi (exact in fp32) times 2^12 rounded to the nearest fp8 e4m3 value (OCP, largest finite 448;
// the product is clamped to +-448 first, since the conversion turns larger values into NaN). The
// value carried is hi + e4m3 * 2^-12: about 15 significant bits, against 11 for hi alone.
constexpr float kLo8Scale = 4096.f;
__device__ __forceinline__ uint32_t lo8_code(float lo) {
    const float s = fminf(fmaxf(lo * kLo8Scale, -448.f), 448.f);
    return (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(s, 0.f, 0, false) & 0xFFu;
}
// Four values at once, packed little-endian (the first value in the low byte).
__device__ __forceinline__ uint32_t lo8_code4(float a, float b, float c, float d) {
    auto cl = [](float v) { return fminf(fmaxf(v * kLo8Scale, -448.f), 448.f); };
    int r = __builtin_amdgcn_cvt_pk_fp8_f32(cl(a), cl(b), 0, false);
    r = __builtin_amdgcn_cvt_pk_fp8_f32(cl(c), cl(d), r, true);
    return (uint32_t)r;
}
__device__ __forceinline__ void split_f16_f8(float v, vsl_half& hi, uint32_t& lo8) {
    hi = (vsl_half)v;
    asm volatile("" : "+v"(hi));
    lo8 = lo8_code(v - (float)hi);
}
// Four consecutive values: hi as four halfs, the four lo8 codes packed (first value in the low byte).
__device__ __forceinline__ void split4_f16_f8(float a, float b, float c, float d, half4& h, uint32_t& lo8) {
    vsl_half h0 = (vsl_half)a, h1 = (vsl_half)b, h2 = (vsl_half)c, h3 = (vsl_half)d;
    asm volatile("" : "+v"(h0), "+v"(h1), "+v"(h2), "+v"(h3));
    h = half4{h0, h1, h2, h3};
    lo8 = lo8_code4(a - (float)h0, b - (float)h1, c - (float)h2, d - (float)h3);
}
// Byte position of column k within its row of the lo8 plane: bits 3 and 4 of k exchanged, so that
// the 16 bytes one lane feeds to v_mfma_scale_f32_32x32x64_f8f6f4 from a 32-column block (columns
// 16t + 8g + e, t = 0, 1, e = 0..7, for lane group g) are contiguous. Groups of four columns
// starting at a multiple of 4 stay contiguous and in order.
__device__ __host__ __forceinline__ constexpr uint32_t lo8_pos(uint32_t k) {
    return (k & ~24u) | ((k & 8u) << 1) | ((k & 16u) >> 1);
}

// Unpack a 16-byte vector of weights into fp32 values.
__device__ __forceinline__ void unpack(const uint4& v, WF16, float* out) {
    const half8 h = __builtin_bit_cast(half8, v);
#pragma unroll
    for (int i = 0; i < 8; ++i) out[i] = (float)h[i];
}
__device__ __forceinline__ void unpack(const uint4& v, WF32, float* out) {
    out[0] = __builtin_bit_cast(float, v.x);
    out[1] = __builtin_bit_cast(float, v.y);
    out[2] = __builtin_bit_cast(float, v.z);
    out[3] = __builtin_bit_cast(float, v.w);
}
// Block-quantized values as stored: Q8 the signed bytes, Q4 the unsigned nibbles (element 2j of a
// byte in the low nibble, 2j + 1 in the high one); the scale / offset are applied by the caller.
__device__ __forceinline__ void unpack(const uint4& v, WQ8, float* out) {
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int k = 0; k < 4; ++k) out[4 * i + k] = (float)(int8_t)(w[i] >> (8 * k));
}
template <class W4>
__device__ __forceinline__ void unpack_q4(const uint4& v, float* out) {
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint32_t lo = w[i] & 0x0F0F0F0Fu, hi = (w[i] >> 4) & 0x0F0F0F0Fu;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            out[8 * i + 2 * k] = (float)((lo >> (8 * k)) & 0xFFu);
            out[8 * i + 2 * k + 1] = (float)((hi >> (8 * k)) & 0xFFu);
        }
    }
}
__device__ __forceinline__ void unpack(const uint4& v, WQ4, float* out) { unpack_q4<WQ4>(v, out); }
__device__ __forceinline__ void unpack(const uint4& v, WQ41, float* out) { unpack_q4<WQ41>(v, out); }

// Butterfly sum across the full wave (every lane ends with the total).
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, VSL_WAVE);
    return v;
}

// Wave-wide sum through DPP lane moves (no LDS round trips): pairs and quads by quad_perm, rows of
// 16 by row rotations, then rows folded by the row-15 / row-31 broadcasts so that lane 63 holds the
// total, which is returned to every lane as a wave-uniform value.
#define VSL_DPP_F(v, ctrl, row_mask) \
    __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), (ctrl), (row_mask), 0xF, false))
__device__ __forceinline__ float wave_sum_dpp(float v) {
    v += VSL_DPP_F(v, 0xB1, 0xF);   // quad_perm [1,0,3,2]
    v += VSL_DPP_F(v, 0x4E, 0xF);   // quad_perm [2,3,0,1]
    v += VSL_DPP_F(v, 0x124, 0xF);  // row_ror:4
    v += VSL_DPP_F(v, 0x128, 0xF);  // row_ror:8
    v += VSL_DPP_F(v, 0x142, 0xA);  // row_bcast:15 into rows 1 and 3
    v += VSL_DPP_F(v, 0x143, 0xC);  // row_bcast:31 into rows 2 and 3
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}
// Wave-wide maximum by the same steps; lanes a broadcast step does not write keep their own value
// (old operand = v), so any set of values, -inf included, reduces correctly.
#define VSL_DPP_M(v, ctrl, row_mask) \
    __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(v), __float_as_int(v), (ctrl), (row_mask), 0xF, false))
__device__ __forceinline__ float wave_max_dpp(float v) {
    v = fmaxf(v, VSL_DPP_M(v, 0xB1, 0xF));
    v = fmaxf(v, VSL_DPP_M(v, 0x4E, 0xF));
    v = fmaxf(v, VSL_DPP_M(v, 0x124, 0xF));
    v = fmaxf(v, VSL_DPP_M(v, 0x128, 0xF));
    v = fmaxf(v, VSL_DPP_M(v, 0x142, 0xA));
    v = fmaxf(v, VSL_DPP_M(v, 0x143, 0xC));
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}
#undef VSL_DPP_M
#undef VSL_DPP_F

// Sum across aligned groups of W = 8 or 16 lanes with DPP row operations (VALU only, every lane of
// the group ends with the sum): quad sums by quad_perm, then the other quad of the half row by
// row_half_mirror (lane i <- 7 - i), then the other half row by row_mirror (lane i <- 15 - i).
template <int W>
__device__ __forceinline__ float group_sum_dpp(float v) {
    static_assert(W == 8 || W == 16, "DPP group sums over 8 or 16 lanes");
    v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0xB1, 0xF, 0xF, false));   // [1,0,3,2]
    v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x4E, 0xF, 0xF, false));   // [2,3,0,1]
    v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x141, 0xF, 0xF, false));  // half mirror
    if constexpr (W == 16)
        v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x140, 0xF, 0xF, false));  // mirror
    return v;
}

// Maximum across aligned rows of 16 lanes, every lane of the row ending with it (the steps of
// group_sum_dpp<16>).
__device__ __forceinline__ float row_max16_dpp(float v) {
    v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0xB1, 0xF, 0xF, false)));
    v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x4E, 0xF, 0xF, false)));
    v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x141, 0xF, 0xF, false)));
    v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x140, 0xF, 0xF, false)));
    return v;
}

// The values of lanes i and i ^ X for X = 8 (row_ror:8 within a 16-lane row), 16 (v_permlane16_swap)
// or 32 (v_permlane32_swap), as an (a, b) pair that is the same in both lanes (a: the lane with the
// X bit clear). VALU only.
template <int X>
__device__ __forceinline__ void lane_pair(float v, float& a, float& b) {
    static_assert(X == 8 || X == 16 || X == 32, "lane pairs at distance 8, 16 or 32");
    if constexpr (X == 8) {
        const float o = __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x128, 0xF, 0xF, false));
        const bool lo = (threadIdx.x & 8) == 0;
        a = lo ? v : o;
        b = lo ? o : v;
    } else {
        const uint32_t u = __float_as_uint(v);
        const auto r = X == 16 ? __builtin_amdgcn_permlane16_swap(u, u, false, false)
                               : __builtin_amdgcn_permlane32_swap(u, u, false, false);
        a = __uint_as_float(r[0]);
        b = __uint_as_float(r[1]);
    }
}

// 2^x by the hardware instruction (no denormal rescaling: results below 2^-126 flush to 0)
__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// Sum across aligned groups of `W` lanes (W a power of two <= 64).
template <int W>
__device__ __forceinline__ float group_sum(float v) {
#pragma unroll
    for (int o = W / 2; o >= 1; o >>= 1) v += __shfl_xor(v, o, VSL_WAVE);
    return v;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, VSL_WAVE));
    return v;
}

// (value, index) argmax with the reference's tie rule: larger value wins, equal values keep the
// lower index (greedy_sampling scans upward with a strict '>').
__device__ __forceinline__ void argmax_merge(float& v, uint32_t& i, float ov, uint32_t oi) {
    if (ov > v || (ov == v && oi < i)) { v = ov; i = oi; }
}

__device__ __forceinline__ void wave_argmax(float& v, uint32_t& i) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) {
        float ov = __shfl_xor(v, o, VSL_WAVE);
        uint32_t oi = __shfl_xor(i, o, VSL_WAVE);
        argmax_merge(v, i, ov, oi);
    }
}

__device__ __forceinline__ float silu(float g) { return g / (1.0f + __expf(-g)); }

// Philox4x32-10 (Salmon et al., SC'11), identical to the host implementation.
__device__ __forceinline__ void philox4x32_10(uint32_t c[4], uint32_t k0, uint32_t k1) {
#pragma unroll
    for (int r = 0; r < 10; ++r) {
        uint64_t p0 = (uint64_t)0xD2511F53u * c[0];
        uint64_t p1 = (uint64_t)0xCD9E8D57u * c[2];
        uint32_t hi0 = (uint32_t)(p0 >> 32), lo0 = (uint32_t)p0;
        uint32_t hi1 = (uint32_t)(p1 >> 32), lo1 = (uint32_t)p1;
        uint32_t n0 = hi1 ^ c[1] ^ k0;
        uint32_t n2 = hi0 ^ c[3] ^ k1;
        c[0] = n0; c[1] = lo1; c[2] = n2; c[3] = lo0;
        k0 += 0x9E3779B9u;
        k1 += 0xBB67AE85u;
    }
}
