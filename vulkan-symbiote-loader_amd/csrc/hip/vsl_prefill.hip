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

// hi/lo split of an fp32 value into two binary16 values (hi + lo carries ~22 significant bits)
__device__ __forceinline__ void split_f16(float v, vsl_half& hi, vsl_half& lo) {
    hi = (vsl_half)v;
    lo = (vsl_half)(v - (float)hi);
}

template <int EPI, bool AX2, bool CX2>
__global__ __launch_bounds__(kGemmThreads) void k_gemm_f16(const vsl_half* __restrict__ A, const vsl_half* __restrict__ B,
                                                           uint32_t M, uint32_t N, uint32_t K, void* __restrict__ C) {
    constexpr int AP = AX2 ? 2 : 1;  // A planes (hi, lo)
    __shared__ __attribute__((aligned(16))) vsl_half As[2][AP][BM * LDS_STRIDE];
    __shared__ __attribute__((aligned(16))) vsl_half Bs[2][BN * LDS_STRIDE];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const uint32_t m0 = blockIdx.y * BM;
    // EPI_SWIGLU: the block covers 64 output columns; B-tile rows 0..63 are gate rows, 64..127 up rows.
    const uint32_t nout0 = blockIdx.x * (EPI == VSL_EPI_SWIGLU ? BN / 2 : BN);
    const size_t plane = (size_t)M * K;

    // global -> register staging: each thread moves 2 x 16 bytes of each A plane and of B per K step
    const int lr = tid >> 2, lk = (tid & 3) * 8;
    auto b_row = [&](int r) -> uint32_t {
        if constexpr (EPI == VSL_EPI_SWIGLU) return r < BN / 2 ? nout0 + r : N + nout0 + (r - BN / 2);
        else return nout0 + r;
    };
    uint4 ra[AP][2], rb[2];
    auto gload = [&](uint32_t k0) {
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const uint32_t r = m0 + lr + i * 64;
#pragma unroll
            for (int p = 0; p < AP; ++p)
                ra[p][i] = r < M ? *reinterpret_cast<const uint4*>(A + p * plane + (size_t)r * K + k0 + lk)
                                 : make_uint4(0, 0, 0, 0);
            rb[i] = *reinterpret_cast<const uint4*>(B + (size_t)b_row(lr + i * 64) * K + k0 + lk);
        }
    };
    auto sstore = [&](int buf) {
#pragma unroll
        for (int i = 0; i < 2; ++i) {
#pragma unroll
            for (int p = 0; p < AP; ++p)
                *reinterpret_cast<uint4*>(&As[buf][p][(lr + i * 64) * LDS_STRIDE + lk]) = ra[p][i];
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
            half8 af[AP][2], bf[2];
#pragma unroll
            for (int p = 0; p < AP; ++p)
#pragma unroll
                for (int i = 0; i < 2; ++i)
                    af[p][i] = *reinterpret_cast<const half8*>(
                        &As[buf][p][(wm * 64 + i * 32 + (lane & 31)) * LDS_STRIDE + kc + (lane >> 5) * 8]);
#pragma unroll
            for (int j = 0; j < 2; ++j)
                bf[j] = *reinterpret_cast<const half8*>(&Bs[buf][(bt[j] + (lane & 31)) * LDS_STRIDE + kc + (lane >> 5) * 8]);
#pragma unroll
            for (int p = 0; p < AP; ++p)
#pragma unroll
                for (int i = 0; i < 2; ++i)
#pragma unroll
                    for (int j = 0; j < 2; ++j)
                        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[p][i], bf[j], acc[i][j], 0, 0, 0);
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
                const float h = silu(acc[i][0][v]) * acc[i][1][v];
                vsl_half* Ch = reinterpret_cast<vsl_half*>(C);
                if constexpr (CX2) {
                    vsl_half hi, lo;
                    split_f16(h, hi, lo);
                    Ch[(size_t)row * N + col] = hi;
                    Ch[(size_t)M * N + (size_t)row * N + col] = lo;
                } else {
                    Ch[(size_t)row * N + col] = (vsl_half)h;
                }
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
template <class KT, bool QX2>
__global__ void k_rope_split(const float* __restrict__ qkv, uint32_t S, uint32_t n_q, uint32_t n_kv, uint32_t hd,
                             uint32_t pos0, const float* __restrict__ rc, const float* __restrict__ rs,
                             vsl_half* __restrict__ q_out, void* __restrict__ kc, void* __restrict__ vc, uint32_t cap) {
    const uint32_t width = (n_q + 2 * n_kv) * hd;  // row length of qkv
    const uint32_t pairs = width / 2;
    const uint64_t total = (uint64_t)S * pairs;
    typedef typename KT::T T;
    const size_t qplane = (size_t)S * n_q * hd;
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
            const size_t o = (size_t)s * qw + col;
            if constexpr (QX2) {
                vsl_half h0, l0, h1, l1;
                split_f16(v0, h0, l0);
                split_f16(v1, h1, l1);
                q_out[o] = h0;
                q_out[o + 1] = h1;
                q_out[qplane + o] = l0;
                q_out[qplane + o + 1] = l1;
            } else {
                q_out[o] = (vsl_half)v0;
                q_out[o + 1] = (vsl_half)v1;
            }
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
template <int HD, bool QX2, bool OX2>
__global__ __launch_bounds__(64) void k_attn_prefill(const vsl_half* __restrict__ q, const vsl_half* __restrict__ kc,
                                                     const vsl_half* __restrict__ vc, uint32_t S, uint32_t pos0,
                                                     uint32_t n_q, uint32_t n_kv, uint32_t cap, float scale,
                                                     vsl_half* __restrict__ out) {
    constexpr int VT_STRIDE = 32 + 8;  // halfs per transposed-V row (one head dim, 32 positions)
    constexpr int QP = QX2 ? 2 : 1;    // q planes; with split q the probabilities are split too
    __shared__ __attribute__((aligned(16))) vsl_half Vt[HD * VT_STRIDE];
    const int lane = threadIdx.x;
    const uint32_t qb = blockIdx.x, h = blockIdx.y;
    const uint32_t kvh = (uint32_t)(((uint64_t)h * n_kv) / n_q);
    const uint32_t s_base = qb * 32;
    const uint32_t my_s = s_base + (lane & 31);  // query row owned by this lane (stats, O^T column)
    const uint32_t qw = n_q * HD;
    const size_t qplane = (size_t)S * qw;
    const float sl2 = scale * 1.4426950408889634f;

    // Q^T as the B operand of S^T = K Q^T: lane holds q row (l%32), hd slots 16c + 8*(l/32)..+7
    half8 qf[QP][HD / 16];
#pragma unroll
    for (int p = 0; p < QP; ++p)
#pragma unroll
        for (int c = 0; c < HD / 16; ++c) {
            if (my_s < S)
                qf[p][c] = *reinterpret_cast<const half8*>(q + p * qplane + (size_t)my_s * qw + (size_t)h * HD + c * 16 +
                                                           (lane >> 5) * 8);
            else
                qf[p][c] = half8{0, 0, 0, 0, 0, 0, 0, 0};
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
#pragma unroll
            for (int p = 0; p < QP; ++p) st = __builtin_amdgcn_mfma_f32_32x32x16_f16(kf, qf[p][c], st, 0, 0, 0);
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
        half8 pf[QP][2];
#pragma unroll
        for (int v = 0; v < 16; ++v) {
            const float pv = (st[v] == -INFINITY) ? 0.f : exp2f(st[v] - mn);
            ps += pv;
            if constexpr (QX2) {
                vsl_half hi, lo;
                split_f16(pv, hi, lo);
                pf[0][v >> 3][v & 7] = hi;
                pf[QP - 1][v >> 3][v & 7] = lo;
            } else {
                pf[0][v >> 3][v & 7] = (vsl_half)pv;
            }
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
#pragma unroll
                for (int p = 0; p < QP; ++p) o[t] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af, pf[p][half_i], o[t], 0, 0, 0);
            }
        }
    }
    if (my_s >= S) return;
    const float inv = l > 0.f ? 1.f / l : 0.f;
    vsl_half* orow = out + (size_t)my_s * qw + (size_t)h * HD;
#pragma unroll
    for (int t = 0; t < HD / 32; ++t)
#pragma unroll
        for (int v = 0; v < 16; ++v) {
            const float val = o[t][v] * inv;
            if constexpr (OX2) {
                vsl_half hi, lo;
                split_f16(val, hi, lo);
                orow[t * 32 + d_row(v, lane)] = hi;
                orow[qplane + t * 32 + d_row(v, lane)] = lo;
            } else {
                orow[t * 32 + d_row(v, lane)] = (vsl_half)val;
            }
        }
}

}  // namespace

template <int EPI>
static void launch_gemm(dim3 grid, hipStream_t s, const vsl_half* a, const vsl_half* b, uint32_t M, uint32_t N,
                        uint32_t K, void* C, bool ax2, bool cx2) {
    if (ax2 && cx2) k_gemm_f16<EPI, true, true><<<grid, kGemmThreads, 0, s>>>(a, b, M, N, K, C);
    else if (ax2) k_gemm_f16<EPI, true, false><<<grid, kGemmThreads, 0, s>>>(a, b, M, N, K, C);
    else if (cx2) k_gemm_f16<EPI, false, true><<<grid, kGemmThreads, 0, s>>>(a, b, M, N, K, C);
    else k_gemm_f16<EPI, false, false><<<grid, kGemmThreads, 0, s>>>(a, b, M, N, K, C);
}

extern "C" int vsl_gemm_f16(const void* A, const void* B, uint32_t M, uint32_t N, uint32_t K, void* C, int epilogue,
                            void* stream) {
    if (!A || !B || !C) return vsl_invalid("vsl_gemm_f16: null pointer");
    if (M == 0) return VSL_OK;
    const bool ax2 = (epilogue & VSL_GEMM_A_X2) != 0, cx2 = (epilogue & VSL_GEMM_C_X2) != 0;
    const int epi = epilogue & 0xFF;
    if (epilogue & ~(0xFF | VSL_GEMM_A_X2 | VSL_GEMM_C_X2)) return vsl_invalid("vsl_gemm_f16: flags 0x%x", epilogue);
    if (cx2 && epi != VSL_EPI_SWIGLU) return vsl_invalid("vsl_gemm_f16: VSL_GEMM_C_X2 needs VSL_EPI_SWIGLU");
    if (K % BK) return vsl_invalid("vsl_gemm_f16: K=%u must be a multiple of %d", K, BK);
    const uint32_t ncols = epi == VSL_EPI_SWIGLU ? BN / 2 : BN;
    if (N % ncols) return vsl_invalid("vsl_gemm_f16: N=%u must be a multiple of %u", N, ncols);
    dim3 grid(N / ncols, (M + BM - 1) / BM);
    hipStream_t s = static_cast<hipStream_t>(stream);
    const vsl_half* a = static_cast<const vsl_half*>(A);
    const vsl_half* b = static_cast<const vsl_half*>(B);
    switch (epi) {
        case VSL_EPI_STORE_F32: launch_gemm<VSL_EPI_STORE_F32>(grid, s, a, b, M, N, K, C, ax2, false); break;
        case VSL_EPI_STORE_F16: launch_gemm<VSL_EPI_STORE_F16>(grid, s, a, b, M, N, K, C, ax2, false); break;
        case VSL_EPI_RESID: launch_gemm<VSL_EPI_RESID>(grid, s, a, b, M, N, K, C, ax2, false); break;
        case VSL_EPI_SWIGLU: launch_gemm<VSL_EPI_SWIGLU>(grid, s, a, b, M, N, K, C, ax2, cx2); break;
        default: return vsl_invalid("vsl_gemm_f16: epilogue %d", epi);
    }
    HIP_TRY(hipGetLastError());
    return VSL_OK;
}

extern "C" int vsl_rope_split_append(const float* qkv, uint32_t S, uint32_t n_q, uint32_t n_kv, uint32_t hd, uint32_t pos0,
                                     const float* rope_cos, const float* rope_sin, void* q_out, int q_dtype,
                                     void* kcache, void* vcache, int kv_dtype, uint32_t cap, void* stream) {
    if (!qkv || !rope_cos || !rope_sin || !q_out || !kcache || !vcache) return vsl_invalid("vsl_rope_split_append: null pointer");
    if (S == 0) return VSL_OK;
    if ((uint64_t)pos0 + S > cap) {
        vsl_set_error("vsl_rope_split_append: positions %u..%u exceed capacity %u", pos0, pos0 + S - 1, cap);
        return VSL_E_CAPACITY;
    }
    if (hd % 2) return vsl_invalid("vsl_rope_split_append: odd head_dim");
    if (q_dtype != VSL_DT_F16 && q_dtype != VSL_DT_F16X2) return vsl_unsupported("vsl_rope_split_append: q dtype %d", q_dtype);
    const uint64_t total = (uint64_t)S * (n_q + 2 * n_kv) * hd / 2;
    const uint32_t grid = (uint32_t)std::min<uint64_t>((total + 255) / 256, 65536);
    hipStream_t s = static_cast<hipStream_t>(stream);
    vsl_half* qo = static_cast<vsl_half*>(q_out);
    const bool x2 = q_dtype == VSL_DT_F16X2;
    if (kv_dtype == VSL_DT_F16) {
        if (x2) k_rope_split<WF16, true><<<grid, 256, 0, s>>>(qkv, S, n_q, n_kv, hd, pos0, rope_cos, rope_sin, qo, kcache, vcache, cap);
        else k_rope_split<WF16, false><<<grid, 256, 0, s>>>(qkv, S, n_q, n_kv, hd, pos0, rope_cos, rope_sin, qo, kcache, vcache, cap);
    } else if (kv_dtype == VSL_DT_F32) {
        if (x2) k_rope_split<WF32, true><<<grid, 256, 0, s>>>(qkv, S, n_q, n_kv, hd, pos0, rope_cos, rope_sin, qo, kcache, vcache, cap);
        else k_rope_split<WF32, false><<<grid, 256, 0, s>>>(qkv, S, n_q, n_kv, hd, pos0, rope_cos, rope_sin, qo, kcache, vcache, cap);
    } else {
        return vsl_unsupported("vsl_rope_split_append: kv dtype %d", kv_dtype);
    }
    HIP_TRY(hipGetLastError());
    return VSL_OK;
}

template <int HD>
static void launch_attn_prefill(dim3 grid, hipStream_t s, const vsl_half* q, const vsl_half* k, const vsl_half* v,
                                uint32_t S, uint32_t pos0, uint32_t n_q, uint32_t n_kv, uint32_t cap, float scale,
                                vsl_half* o, bool qx2, bool ox2) {
    if (qx2 && ox2) k_attn_prefill<HD, true, true><<<grid, 64, 0, s>>>(q, k, v, S, pos0, n_q, n_kv, cap, scale, o);
    else if (qx2) k_attn_prefill<HD, true, false><<<grid, 64, 0, s>>>(q, k, v, S, pos0, n_q, n_kv, cap, scale, o);
    else if (ox2) k_attn_prefill<HD, false, true><<<grid, 64, 0, s>>>(q, k, v, S, pos0, n_q, n_kv, cap, scale, o);
    else k_attn_prefill<HD, false, false><<<grid, 64, 0, s>>>(q, k, v, S, pos0, n_q, n_kv, cap, scale, o);
}

extern "C" int vsl_attn_prefill(const void* q, int q_dtype, const void* kcache, const void* vcache, uint32_t S,
                                uint32_t pos0, uint32_t n_q, uint32_t n_kv, uint32_t hd, uint32_t cap, float scale,
                                void* out, int out_dtype, void* stream) {
    if (!q || !kcache || !vcache || !out) return vsl_invalid("vsl_attn_prefill: null pointer");
    if (S == 0) return VSL_OK;
    if (n_kv == 0 || n_q % n_kv) return vsl_invalid("vsl_attn_prefill: n_q=%u n_kv=%u", n_q, n_kv);
    if ((uint64_t)pos0 + S > cap) {
        vsl_set_error("vsl_attn_prefill: positions %u..%u exceed capacity %u", pos0, pos0 + S - 1, cap);
        return VSL_E_CAPACITY;
    }
    if ((q_dtype != VSL_DT_F16 && q_dtype != VSL_DT_F16X2) || (out_dtype != VSL_DT_F16 && out_dtype != VSL_DT_F16X2))
        return vsl_unsupported("vsl_attn_prefill: dtypes %d/%d", q_dtype, out_dtype);
    dim3 grid((S + 31) / 32, n_q);
    hipStream_t s = static_cast<hipStream_t>(stream);
    const bool qx2 = q_dtype == VSL_DT_F16X2, ox2 = out_dtype == VSL_DT_F16X2;
    const vsl_half* qq = static_cast<const vsl_half*>(q);
    const vsl_half* kk = static_cast<const vsl_half*>(kcache);
    const vsl_half* vv = static_cast<const vsl_half*>(vcache);
    vsl_half* oo = static_cast<vsl_half*>(out);
    if (hd == 128)
        launch_attn_prefill<128>(grid, s, qq, kk, vv, S, pos0, n_q, n_kv, cap, scale, oo, qx2, ox2);
    else if (hd == 64)
        launch_attn_prefill<64>(grid, s, qq, kk, vv, S, pos0, n_q, n_kv, cap, scale, oo, qx2, ox2);
    else
        return vsl_unsupported("vsl_attn_prefill: head_dim %u", hd);
    HIP_TRY(hipGetLastError());
    return VSL_OK;
}
