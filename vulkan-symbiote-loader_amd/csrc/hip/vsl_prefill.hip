// vsl_prefill.hip -- prefill (S positions at once) on gfx950 MFMA.
//
// k_gemm_f16:      C[M][N] = A[M][K] * B[N][K]^T with v_mfma_f32_32x32x16_f16, 128x128 block tile,
//                  BK = 32, LDS double buffering, fused epilogues (fp32 / fp16 store, residual add,
//                  SwiGLU over [Wgate; Wup]).
// k_rope_split:    QKV GEMM output -> RoPE(q, k) at positions pos0+s -> q (fp16), K/V cache (fp16).
// k_attn_prefill:  causal flash attention, one wavefront per (32 query rows, query head), computing
//                  S^T = K Q^T and O^T = V^T P^T on MFMA so that every lane owns one query row's
//                  softmax statistics and output column.
//
// MFMA 32x32x16 f16 operand layout used here (lane l of a 64-lane wave):
//   A (32 x 16): row l%32, 8 consecutive k-slots 8*(l/32)..+7
//   B (16 x 32): col l%32, the same 8 k-slots
//   D (32 x 32): 16 floats; element v is row (v/4)*8 + (l/32)*4 + v%4, col l%32
// Which physical k a slot holds is free as long as A and B agree.
#include <hip/hip_runtime.h>

#include <cmath>

#include "vsl_device.h"
#include "vsl_hip.h"
#include "vsl_internal.h"

namespace {

constexpr int kGemmThreads = 256;
constexpr int BM = 128, BN = 128, BK = 32, LDS_STRIDE = BK + 8;  // halfs per LDS row (80 bytes)

__device__ __forceinline__ int d_row(int v, int lane) { return (v >> 2) * 8 + (lane >> 5) * 4 + (v & 3); }

template <int EPI>
__global__ __launch_bounds__(kGemmThreads) void k_gemm_f16(const vsl_half* __restrict__ A, const vsl_half* __restrict__ B,
                                                           uint32_t M, uint32_t N, uint32_t K, void* __restrict__ C) {
    __shared__ __attribute__((aligned(16))) vsl_half As[2][BM * LDS_STRIDE];
    __shared__ __attribute__((aligned(16))) vsl_half Bs[2][BN * LDS_STRIDE];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const uint32_t m0 = blockIdx.y * BM;
    // EPI_SWIGLU: the block covers 64 output columns; B-tile rows 0..63 are gate rows, 64..127 up rows.
    const uint32_t nout0 = blockIdx.x * (EPI == VSL_EPI_SWIGLU ? BN / 2 : BN);

    // global -> register staging: each thread moves 2 x 16 bytes of A and of B per K step
    const int lr = tid >> 2, lk = (tid & 3) * 8;
    auto b_row = [&](int r) -> uint32_t {
        if constexpr (EPI == VSL_EPI_SWIGLU) return r < BN / 2 ? nout0 + r : N + nout0 + (r - BN / 2);
        else return nout0 + r;
    };
    uint4 ra[2], rb[2];
    auto gload = [&](uint32_t k0) {
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const uint32_t r = m0 + lr + i * 64;
            ra[i] = r < M ? *reinterpret_cast<const uint4*>(A + (size_t)r * K + k0 + lk) : make_uint4(0, 0, 0, 0);
            rb[i] = *reinterpret_cast<const uint4*>(B + (size_t)b_row(lr + i * 64) * K + k0 + lk);
        }
    };
    auto sstore = [&](int buf) {
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            *reinterpret_cast<uint4*>(&As[buf][(lr + i * 64) * LDS_STRIDE + lk]) = ra[i];
            *reinterpret_cast<uint4*>(&Bs[buf][(lr + i * 64) * LDS_STRIDE + lk]) = rb[i];
        }
    };

    float16v acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.f;

    // B-tile rows of this wave's two 32-column tiles
    int bt[2];
    if constexpr (EPI == VSL_EPI_SWIGLU) {
        bt[0] = wn * 32;
        bt[1] = BN / 2 + wn * 32;
    } else {
        bt[0] = wn * 64;
        bt[1] = wn * 64 + 32;
    }

    const uint32_t nk = K / BK;
    gload(0);
    sstore(0);
    __syncthreads();
    for (uint32_t kt = 0; kt < nk; ++kt) {
        const int buf = kt & 1;
        if (kt + 1 < nk) gload((kt + 1) * BK);
#pragma unroll
        for (int kc = 0; kc < BK; kc += 16) {
            half8 af[2], bf[2];
#pragma unroll
            for (int i = 0; i < 2; ++i)
                af[i] = *reinterpret_cast<const half8*>(&As[buf][(wm * 64 + i * 32 + (lane & 31)) * LDS_STRIDE + kc + (lane >> 5) * 8]);
#pragma unroll
            for (int j = 0; j < 2; ++j)
                bf[j] = *reinterpret_cast<const half8*>(&Bs[buf][(bt[j] + (lane & 31)) * LDS_STRIDE + kc + (lane >> 5) * 8]);
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int j = 0; j < 2; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[i], bf[j], acc[i][j], 0, 0, 0);
        }
        if (kt + 1 < nk) sstore(buf ^ 1);
        __syncthreads();
    }

    // epilogue
#pragma unroll
    for (int i = 0; i < 2; ++i) {
#pragma unroll
        for (int v = 0; v < 16; ++v) {
            const uint32_t row = m0 + wm * 64 + i * 32 + d_row(v, lane);
            if (row >= M) continue;
            if constexpr (EPI == VSL_EPI_SWIGLU) {
                const uint32_t col = nout0 + wn * 32 + (lane & 31);
                const float g = acc[i][0][v], u = acc[i][1][v];
                reinterpret_cast<vsl_half*>(C)[(size_t)row * N + col] = (vsl_half)(silu(g) * u);
            } else {
#pragma unroll
                for (int j = 0; j < 2; ++j) {
                    const uint32_t col = nout0 + wn * 64 + j * 32 + (lane & 31);
                    const size_t o = (size_t)row * N + col;
                    if constexpr (EPI == VSL_EPI_STORE_F32) reinterpret_cast<float*>(C)[o] = acc[i][j][v];
                    else if constexpr (EPI == VSL_EPI_STORE_F16) reinterpret_cast<vsl_half*>(C)[o] = (vsl_half)acc[i][j][v];
                    else reinterpret_cast<float*>(C)[o] += acc[i][j][v];
                }
            }
        }
    }
}

// ---------------------------------------------------------------------------------------------
// RoPE + split of the prefill QKV projection
// ---------------------------------------------------------------------------------------------
template <class KT>
__global__ void k_rope_split(const float* __restrict__ qkv, uint32_t S, uint32_t n_q, uint32_t n_kv, uint32_t hd,
                             uint32_t pos0, const float* __restrict__ rc, const float* __restrict__ rs,
                             vsl_half* __restrict__ q_out, void* __restrict__ kc, void* __restrict__ vc, uint32_t cap) {
    const uint32_t width = (n_q + 2 * n_kv) * hd;  // row length of qkv
    const uint32_t pairs = width / 2;
    const uint64_t total = (uint64_t)S * pairs;
    typedef typename KT::T T;
    for (uint64_t e = blockIdx.x * (uint64_t)blockDim.x + threadIdx.x; e < total; e += (uint64_t)gridDim.x * blockDim.x) {
        const uint32_t s = (uint32_t)(e / pairs), pr = (uint32_t)(e % pairs);
        const uint32_t col = pr * 2;
        const uint32_t pos = pos0 + s;
        float v0 = qkv[(size_t)s * width + col], v1 = qkv[(size_t)s * width + col + 1];
        const uint32_t qw = n_q * hd, kw = n_kv * hd;
        if (col < qw + kw) {
            const uint32_t j = (col % hd) >> 1;
            const float c = rc[(size_t)pos * (hd >> 1) + j], sn = rs[(size_t)pos * (hd >> 1) + j];
            const float a = v0 * c - v1 * sn, b = v0 * sn + v1 * c;
            v0 = a;
            v1 = b;
        }
        if (col < qw) {
            q_out[(size_t)s * qw + col] = (vsl_half)v0;
            q_out[(size_t)s * qw + col + 1] = (vsl_half)v1;
        } else {
            const bool is_k = col < qw + kw;
            const uint32_t cc = col - (is_k ? qw : qw + kw);
            const uint32_t kvh = cc / hd, dim = cc % hd;
            T* dst = static_cast<T*>(is_k ? kc : vc) + ((size_t)kvh * cap + pos) * hd + dim;
            store_elem(dst, v0);
            store_elem(dst + 1, v1);
        }
    }
}

// ---------------------------------------------------------------------------------------------
// causal flash attention (prefill), fp16 in / fp16 out, fp32 softmax statistics
// ---------------------------------------------------------------------------------------------
template <int HD>
__global__ __launch_bounds__(64) void k_attn_prefill(const vsl_half* __restrict__ q, const vsl_half* __restrict__ kc,
                                                     const vsl_half* __restrict__ vc, uint32_t S, uint32_t pos0,
                                                     uint32_t n_q, uint32_t n_kv, uint32_t cap, float scale,
                                                     vsl_half* __restrict__ out) {
    constexpr int VT_STRIDE = 32 + 8;  // halfs per transposed-V row (one head dim, 32 positions)
    __shared__ __attribute__((aligned(16))) vsl_half Vt[HD * VT_STRIDE];
    const int lane = threadIdx.x;
    const uint32_t qb = blockIdx.x, h = blockIdx.y;
    const uint32_t kvh = (uint32_t)(((uint64_t)h * n_kv) / n_q);
    const uint32_t s_base = qb * 32;
    const uint32_t my_s = s_base + (lane & 31);  // query row owned by this lane (stats, O^T column)
    const uint32_t qw = n_q * HD;
    const float sl2 = scale * 1.4426950408889634f;

    // Q^T as the B operand of S^T = K Q^T: lane holds q row (l%32), hd slots 16c + 8*(l/32)..+7
    half8 qf[HD / 16];
#pragma unroll
    for (int c = 0; c < HD / 16; ++c) {
        if (my_s < S)
            qf[c] = *reinterpret_cast<const half8*>(q + (size_t)my_s * qw + (size_t)h * HD + c * 16 + (lane >> 5) * 8);
        else
            qf[c] = half8{0, 0, 0, 0, 0, 0, 0, 0};
    }
    float16v o[HD / 32];
#pragma unroll
    for (int t = 0; t < HD / 32; ++t)
#pragma unroll
        for (int v = 0; v < 16; ++v) o[t][v] = 0.f;
    float m = -INFINITY, l = 0.f;

    const uint32_t last_s = min(S, s_base + 32) - 1;
    const uint32_t kv_end = pos0 + last_s + 1;  // positions 0..kv_end-1 are visible to some row
    const vsl_half* Kb = kc + (size_t)kvh * cap * HD;
    const vsl_half* Vb = vc + (size_t)kvh * cap * HD;
    const uint32_t my_pos = pos0 + my_s;

    for (uint32_t t0 = 0; t0 < kv_end; t0 += 32) {
        // stage V^T for positions t0..t0+31 (zero beyond kv_end)
        __syncthreads();
        for (int e = lane; e < 32 * (HD / 8); e += 64) {
            const int r = e / (HD / 8), c8 = (e % (HD / 8)) * 8;
            half8 vv = (t0 + r < kv_end) ? *reinterpret_cast<const half8*>(Vb + (size_t)(t0 + r) * HD + c8)
                                         : half8{0, 0, 0, 0, 0, 0, 0, 0};
#pragma unroll
            for (int i = 0; i < 8; ++i) Vt[(c8 + i) * VT_STRIDE + r] = vv[i];
        }
        // S^T[kv][q] = sum_d K[kv][d] Q[q][d]
        float16v st;
#pragma unroll
        for (int v = 0; v < 16; ++v) st[v] = 0.f;
        const uint32_t krow = t0 + (lane & 31);
#pragma unroll
        for (int c = 0; c < HD / 16; ++c) {
            half8 kf = krow < kv_end ? *reinterpret_cast<const half8*>(Kb + (size_t)krow * HD + c * 16 + (lane >> 5) * 8)
                                     : half8{0, 0, 0, 0, 0, 0, 0, 0};
            st = __builtin_amdgcn_mfma_f32_32x32x16_f16(kf, qf[c], st, 0, 0, 0);
        }
        // causal mask + online softmax over this lane's 16 kv values of its query row
        float bm = -INFINITY;
#pragma unroll
        for (int v = 0; v < 16; ++v) {
            const uint32_t kvp = t0 + d_row(v, lane);
            const float sc = (kvp <= my_pos && kvp < kv_end) ? st[v] * sl2 : -INFINITY;
            st[v] = sc;
            bm = fmaxf(bm, sc);
        }
        bm = fmaxf(bm, __shfl_xor(bm, 32, 64));
        const float mn = fmaxf(m, bm);
        const float corr = (mn == -INFINITY) ? 1.f : exp2f(m - mn);
        float ps = 0.f;
        half8 pf[2];
#pragma unroll
        for (int v = 0; v < 16; ++v) {
            const float p = (st[v] == -INFINITY) ? 0.f : exp2f(st[v] - mn);
            ps += p;
            pf[v >> 3][v & 7] = (vsl_half)p;
        }
        ps += __shfl_xor(ps, 32, 64);
        l = l * corr + ps;
        m = mn;
#pragma unroll
        for (int t = 0; t < HD / 32; ++t)
#pragma unroll
            for (int v = 0; v < 16; ++v) o[t][v] *= corr;
        __syncthreads();
        // O^T[dim][q] += sum_kv V^T[dim][kv] P^T[kv][q]; k-slots: v=0..7 -> MFMA 0, v=8..15 -> MFMA 1
#pragma unroll
        for (int t = 0; t < HD / 32; ++t) {
            const int dim = t * 32 + (lane & 31);
#pragma unroll
            for (int half_i = 0; half_i < 2; ++half_i) {
                // kv positions of slots v = 8*half_i + 0..7: rows d_row(v) = (v/4)*8 + (l/32)*4 + v%4
                const int r0 = (half_i * 2) * 8 + (lane >> 5) * 4;
                const int r1 = (half_i * 2 + 1) * 8 + (lane >> 5) * 4;
                half4 a0 = *reinterpret_cast<const half4*>(&Vt[dim * VT_STRIDE + r0]);
                half4 a1 = *reinterpret_cast<const half4*>(&Vt[dim * VT_STRIDE + r1]);
                half8 af = half8{a0[0], a0[1], a0[2], a0[3], a1[0], a1[1], a1[2], a1[3]};
                o[t] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af, pf[half_i], o[t], 0, 0, 0);
            }
        }
    }
    if (my_s >= S) return;
    const float inv = l > 0.f ? 1.f / l : 0.f;
    vsl_half* orow = out + (size_t)my_s * qw + (size_t)h * HD;
#pragma unroll
    for (int t = 0; t < HD / 32; ++t)
#pragma unroll
        for (int v = 0; v < 16; ++v) orow[t * 32 + d_row(v, lane)] = (vsl_half)(o[t][v] * inv);
}

}  // namespace

extern "C" int vsl_gemm_f16(const void* A, const void* B, uint32_t M, uint32_t N, uint32_t K, void* C, int epilogue,
                            void* stream) {
    if (!A || !B || !C) return vsl_invalid("vsl_gemm_f16: null pointer");
    if (M == 0) return VSL_OK;
    if (K % BK) return vsl_invalid("vsl_gemm_f16: K=%u must be a multiple of %d", K, BK);
    const uint32_t ncols = epilogue == VSL_EPI_SWIGLU ? BN / 2 : BN;
    if (N % ncols) return vsl_invalid("vsl_gemm_f16: N=%u must be a multiple of %u", N, ncols);
    dim3 grid(N / ncols, (M + BM - 1) / BM);
    hipStream_t s = static_cast<hipStream_t>(stream);
    const vsl_half* a = static_cast<const vsl_half*>(A);
    const vsl_half* b = static_cast<const vsl_half*>(B);
    switch (epilogue) {
        case VSL_EPI_STORE_F32: k_gemm_f16<VSL_EPI_STORE_F32><<<grid, kGemmThreads, 0, s>>>(a, b, M, N, K, C); break;
        case VSL_EPI_STORE_F16: k_gemm_f16<VSL_EPI_STORE_F16><<<grid, kGemmThreads, 0, s>>>(a, b, M, N, K, C); break;
        case VSL_EPI_RESID: k_gemm_f16<VSL_EPI_RESID><<<grid, kGemmThreads, 0, s>>>(a, b, M, N, K, C); break;
        case VSL_EPI_SWIGLU: k_gemm_f16<VSL_EPI_SWIGLU><<<grid, kGemmThreads, 0, s>>>(a, b, M, N, K, C); break;
        default: return vsl_invalid("vsl_gemm_f16: epilogue %d", epilogue);
    }
    HIP_TRY(hipGetLastError());
    return VSL_OK;
}

extern "C" int vsl_rope_split_append(const float* qkv, uint32_t S, uint32_t n_q, uint32_t n_kv, uint32_t hd, uint32_t pos0,
                                     const float* rope_cos, const float* rope_sin, void* q_out, void* kcache, void* vcache,
                                     int kv_dtype, uint32_t cap, void* stream) {
    if (!qkv || !rope_cos || !rope_sin || !q_out || !kcache || !vcache) return vsl_invalid("vsl_rope_split_append: null pointer");
    if (S == 0) return VSL_OK;
    if ((uint64_t)pos0 + S > cap) return vsl_set_error("vsl_rope_split_append: positions exceed capacity"), VSL_E_CAPACITY;
    if (hd % 2) return vsl_invalid("vsl_rope_split_append: odd head_dim");
    const uint64_t total = (uint64_t)S * (n_q + 2 * n_kv) * hd / 2;
    const uint32_t grid = (uint32_t)std::min<uint64_t>((total + 255) / 256, 65536);
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (kv_dtype == VSL_DT_F16)
        k_rope_split<WF16><<<grid, 256, 0, s>>>(qkv, S, n_q, n_kv, hd, pos0, rope_cos, rope_sin,
                                               static_cast<vsl_half*>(q_out), kcache, vcache, cap);
    else if (kv_dtype == VSL_DT_F32)
        k_rope_split<WF32><<<grid, 256, 0, s>>>(qkv, S, n_q, n_kv, hd, pos0, rope_cos, rope_sin,
                                               static_cast<vsl_half*>(q_out), kcache, vcache, cap);
    else
        return vsl_unsupported("vsl_rope_split_append: kv dtype %d", kv_dtype);
    HIP_TRY(hipGetLastError());
    return VSL_OK;
}

extern "C" int vsl_attn_prefill(const void* q, const void* kcache, const void* vcache, uint32_t S, uint32_t pos0,
                                uint32_t n_q, uint32_t n_kv, uint32_t hd, uint32_t cap, float scale, void* out,
                                void* stream) {
    if (!q || !kcache || !vcache || !out) return vsl_invalid("vsl_attn_prefill: null pointer");
    if (S == 0) return VSL_OK;
    if (n_kv == 0 || n_q % n_kv) return vsl_invalid("vsl_attn_prefill: n_q=%u n_kv=%u", n_q, n_kv);
    if ((uint64_t)pos0 + S > cap) return vsl_set_error("vsl_attn_prefill: positions exceed capacity"), VSL_E_CAPACITY;
    dim3 grid((S + 31) / 32, n_q);
    hipStream_t s = static_cast<hipStream_t>(stream);
    const vsl_half* qq = static_cast<const vsl_half*>(q);
    const vsl_half* kk = static_cast<const vsl_half*>(kcache);
    const vsl_half* vv = static_cast<const vsl_half*>(vcache);
    vsl_half* oo = static_cast<vsl_half*>(out);
    if (hd == 128)
        k_attn_prefill<128><<<grid, 64, 0, s>>>(qq, kk, vv, S, pos0, n_q, n_kv, cap, scale, oo);
    else if (hd == 64)
        k_attn_prefill<64><<<grid, 64, 0, s>>>(qq, kk, vv, S, pos0, n_q, n_kv, cap, scale, oo);
    else
        return vsl_unsupported("vsl_attn_prefill: head_dim %u", hd);
    HIP_TRY(hipGetLastError());
    return VSL_OK;
}
