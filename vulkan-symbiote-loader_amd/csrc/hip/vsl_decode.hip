// vsl_decode.hip -- bs=1 decode kernels for gfx950.
//
// Every decode-step GEMV is HBM-bound (1 flop/byte): the kernels stream each weight row once with
// 16-byte loads, keep the (normalised) activation vector in LDS as fp32, reduce across the 64-lane
// wavefront with butterfly shuffles, and fuse the neighbouring elementwise op into the epilogue:
//   k_gemv_dec<EPI_QKV>    RMSNorm -> [Wq;Wk;Wv] -> RoPE -> q + KV-cache append
//   k_gemv_dec<EPI_RESID>  W_o / W_down -> residual add
//   k_gemv_dec<EPI_SWIGLU> RMSNorm -> [Wgate;Wup] -> silu(g)*u
//   k_gemv_dec<EPI_ARGMAX> final RMSNorm -> W_out -> logits + fused greedy argmax + next embedding
// and k_attn_decode is a split-KV flash-decode kernel with an in-kernel combine.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdio>

#include "vsl_device.h"
#include "vsl_hip.h"
#include "vsl_internal.h"

namespace {

constexpr int kBlock = 256;
constexpr int kWaves = kBlock / VSL_WAVE;
constexpr uint32_t kMaxLmBlocks = 1024;

enum Epi { EPI_STORE = 0, EPI_RESID = 1, EPI_SWIGLU = 2, EPI_QKV = 3, EPI_ARGMAX = 4, EPI_STORE_F16 = 5 };

struct GemvArgs {
    const void* W;
    uint32_t N;  // output rows (EPI_SWIGLU: F, the weight holds 2F rows)
    uint32_t K;
    const float* x;
    const float* gamma;  // RMSNorm gains; nullptr = no norm prologue
    float eps;
    float* y;
    // EPI_QKV
    uint32_t n_q, n_kv, hd, cap;
    const float* rope_cos;
    const float* rope_sin;
    void* kc;
    void* vc;
    float* q_out;
    // EPI_ARGMAX
    float* ws_val;
    uint32_t* ws_idx;
    uint32_t* tokens;
    const void* embed;
    float* x_next;
    vsl_ctrl* ctrl;
};

// ---------------------------------------------------------------------------------------------
// activation staging (optionally RMS-normalised, rms_norm.comp:24-34)
// ---------------------------------------------------------------------------------------------
__device__ __forceinline__ void stage_x(const float* __restrict__ x, const float* __restrict__ gamma, float eps,
                                        uint32_t K, float* __restrict__ xs, float* red) {
    const uint32_t tid = threadIdx.x;
    float ss = 0.f;
    for (uint32_t i = tid * 4; i < K; i += kBlock * 4) {
        float4 v = *reinterpret_cast<const float4*>(x + i);
        *reinterpret_cast<float4*>(xs + i) = v;
        ss += v.x * v.x + v.y * v.y + v.z * v.z + v.w * v.w;
    }
    if (gamma) {
        ss = wave_sum(ss);
        if ((tid & 63) == 0) red[tid >> 6] = ss;
        __syncthreads();
        float tot = 0.f;
#pragma unroll
        for (int w = 0; w < kWaves; ++w) tot += red[w];
        const float inv = 1.0f / sqrtf(tot / (float)K + eps);
        for (uint32_t i = tid * 4; i < K; i += kBlock * 4) {
            float4 v = *reinterpret_cast<float4*>(xs + i);
            float4 g = *reinterpret_cast<const float4*>(gamma + i);
            v.x = v.x * inv * g.x;
            v.y = v.y * inv * g.y;
            v.z = v.z * inv * g.z;
            v.w = v.w * inv * g.w;
            *reinterpret_cast<float4*>(xs + i) = v;
        }
    }
    __syncthreads();
}

template <class WT>
__device__ __forceinline__ void load_x(const float* xs, uint32_t kk, float* xv) {
    if constexpr (WT::kVec == 8) {
        float4 a = *reinterpret_cast<const float4*>(xs + kk);
        float4 b = *reinterpret_cast<const float4*>(xs + kk + 4);
        xv[0] = a.x; xv[1] = a.y; xv[2] = a.z; xv[3] = a.w;
        xv[4] = b.x; xv[5] = b.y; xv[6] = b.z; xv[7] = b.w;
    } else {
        float4 a = *reinterpret_cast<const float4*>(xs + kk);
        xv[0] = a.x; xv[1] = a.y; xv[2] = a.z; xv[3] = a.w;
    }
}

// The sampled token's bookkeeping, run by the single block that finished last:
// tokens[step] = tok; x_next = embed[tok] (the next step's embedding_lookup); pos++, step++.
template <class ET>
__device__ void finish_token(uint32_t tok, uint32_t V, uint32_t d, const void* embed, float* x_next,
                             uint32_t* tokens, vsl_ctrl* ctrl) {
    const uint32_t tid = threadIdx.x;
    const uint32_t row = tok < V ? tok : V - 1;  // embedding_lookup.comp:32
    constexpr int VEC = ET::kVec;              // d % 8 == 0: whole 16-byte vectors
    const typename ET::T* e = static_cast<const typename ET::T*>(embed) + (size_t)row * d;
    for (uint32_t i = tid * VEC; i < d; i += blockDim.x * VEC) {
        float f[VEC];
        unpack(load16<false>(e + i), ET(), f);
#pragma unroll
        for (int j = 0; j < VEC; j += 4)
            *reinterpret_cast<float4*>(x_next + i + j) = make_float4(f[j], f[j + 1], f[j + 2], f[j + 3]);
    }
    if (tid == 0) {
        const uint32_t step = ctrl->step;
        tokens[step] = tok;
        ctrl->token = tok;
        ctrl->step = step + 1;
        ctrl->pos = ctrl->pos + 1;
        if (step + 1 >= ctrl->max_steps || (ctrl->stop_on_eos && (tok == 0u || tok == 2u))) ctrl->done = 1u;
    }
}

// ---------------------------------------------------------------------------------------------
// decode GEMV
// ---------------------------------------------------------------------------------------------
template <class WT, int R, int U, int EPI, class ET>
__global__ __launch_bounds__(kBlock) void k_gemv_dec(GemvArgs a) {
    __shared__ float red[kWaves];
    __shared__ float bval[kWaves];
    __shared__ uint32_t bidx[kWaves];
    extern __shared__ float xs[];

    uint32_t pos = 0;
    if (a.ctrl) {
        if (a.ctrl->done) return;
        pos = a.ctrl->pos;
        if constexpr (EPI == EPI_QKV) {
            if (pos >= a.cap) {
                if (blockIdx.x == 0 && threadIdx.x == 0) { a.ctrl->error = 1u; a.ctrl->done = 1u; }
                return;
            }
        }
    }
    stage_x(a.x, a.gamma, a.eps, a.K, xs, red);

    typedef typename WT::T T;
    constexpr int VEC = WT::kVec;
    constexpr uint32_t SPAN = 64 * VEC;
    const T* __restrict__ W = static_cast<const T*>(a.W);
    const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    constexpr int RG = (EPI == EPI_SWIGLU) ? R / 2 : R;  // logical rows per group
    const uint32_t n_groups = (a.N + RG - 1) / RG;

    float best_v = -INFINITY;
    uint32_t best_i = 0xFFFFFFFFu;

    for (uint32_t g = blockIdx.x * kWaves + wave; g < n_groups; g += gridDim.x * kWaves) {
        uint32_t rows[R];
        bool ok[R];
#pragma unroll
        for (int r = 0; r < R; ++r) {
            if constexpr (EPI == EPI_SWIGLU) {
                const uint32_t lr = g * RG + (r % RG);
                ok[r] = lr < a.N;
                rows[r] = (r < RG) ? lr : a.N + lr;
            } else {
                rows[r] = g * R + r;
                ok[r] = rows[r] < a.N;
            }
        }
        float acc[R];
#pragma unroll
        for (int r = 0; r < R; ++r) acc[r] = 0.f;

        for (uint32_t k0 = 0; k0 < a.K; k0 += SPAN * U) {
            uint4 w[R][U];
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const uint32_t kk = k0 + u * SPAN + lane * VEC;
#pragma unroll
                for (int r = 0; r < R; ++r) {
                    if (ok[r] && kk < a.K)
                        w[r][u] = load16<true>(W + (size_t)rows[r] * a.K + kk);
                    else
                        w[r][u] = make_uint4(0u, 0u, 0u, 0u);
                }
            }
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const uint32_t kk = k0 + u * SPAN + lane * VEC;
                if (kk < a.K) {
                    float xv[VEC];
                    load_x<WT>(xs, kk, xv);
#pragma unroll
                    for (int r = 0; r < R; ++r) {
                        float wf[VEC];
                        unpack(w[r][u], WT(), wf);
#pragma unroll
                        for (int i = 0; i < VEC; ++i) acc[r] = fmaf(wf[i], xv[i], acc[r]);
                    }
                }
            }
        }
#pragma unroll
        for (int r = 0; r < R; ++r) acc[r] = wave_sum(acc[r]);

        if constexpr (EPI == EPI_STORE) {
            if (lane == 0) {
#pragma unroll
                for (int r = 0; r < R; ++r)
                    if (ok[r]) a.y[rows[r]] = acc[r];
            }
        } else if constexpr (EPI == EPI_STORE_F16) {
            if (lane == 0) {
#pragma unroll
                for (int r = 0; r < R; ++r)
                    if (ok[r]) reinterpret_cast<vsl_half*>(a.y)[rows[r]] = (vsl_half)acc[r];
            }
        } else if constexpr (EPI == EPI_RESID) {
            if (lane == 0) {
#pragma unroll
                for (int r = 0; r < R; ++r)
                    if (ok[r]) a.y[rows[r]] += acc[r];
            }
        } else if constexpr (EPI == EPI_SWIGLU) {
            if (lane == 0) {
#pragma unroll
                for (int r = 0; r < RG; ++r)
                    if (ok[r]) a.y[rows[r]] = silu(acc[r]) * acc[r + RG];
            }
        } else if constexpr (EPI == EPI_QKV) {
            static_assert(R % 2 == 0, "QKV groups hold whole RoPE pairs");
            if (lane == 0) {
                const uint32_t qrows = a.n_q * a.hd, krows = a.n_kv * a.hd;
#pragma unroll
                for (int r = 0; r < R; r += 2) {
                    if (!ok[r]) continue;
                    const uint32_t row = rows[r];
                    float v0 = acc[r], v1 = acc[r + 1];
                    if (row < qrows + krows) {  // RoPE on q and k (adjacent pair row, row+1)
                        const uint32_t j = (row % a.hd) >> 1;
                        const float c = a.rope_cos[(size_t)pos * (a.hd >> 1) + j];
                        const float s = a.rope_sin[(size_t)pos * (a.hd >> 1) + j];
                        const float r0 = v0 * c - v1 * s;
                        const float r1 = v0 * s + v1 * c;
                        v0 = r0;
                        v1 = r1;
                    }
                    if (row < qrows) {
                        a.q_out[row] = v0;
                        a.q_out[row + 1] = v1;
                    } else {
                        const bool is_k = row < qrows + krows;
                        const uint32_t rr = row - (is_k ? qrows : qrows + krows);
                        const uint32_t kvh = rr / a.hd, dim = rr % a.hd;
                        const size_t off = ((size_t)kvh * a.cap + pos) * a.hd + dim;
                        typedef typename ET::T KT;
                        KT* dst = static_cast<KT*>(is_k ? a.kc : a.vc);
                        store_elem(dst + off, v0);
                        store_elem(dst + off + 1, v1);
                    }
                }
            }
        } else if constexpr (EPI == EPI_ARGMAX) {
#pragma unroll
            for (int r = 0; r < R; ++r) {
                if (ok[r]) {
                    if (lane == 0) a.y[rows[r]] = acc[r];
                    argmax_merge(best_v, best_i, acc[r], rows[r]);
                }
            }
        }
    }

    if constexpr (EPI == EPI_ARGMAX) {
        // per-block partial argmax; k_argmax_finish reduces the partials in the next launch (a
        // kernel boundary is the cheapest cross-block visibility point on this chip)
        if (lane == 0) {
            bval[wave] = best_v;
            bidx[wave] = best_i;
        }
        __syncthreads();
        if (threadIdx.x == 0) {
            float v = bval[0];
            uint32_t i = bidx[0];
#pragma unroll
            for (int w = 1; w < kWaves; ++w) argmax_merge(v, i, bval[w], bidx[w]);
            a.ws_val[blockIdx.x] = v;
            a.ws_idx[blockIdx.x] = i;
        }
    }
}

// Final greedy reduction over the lm_head blocks' partials, then the token bookkeeping.
constexpr int kFinishThreads = 1024;
template <class ET>
__global__ __launch_bounds__(kFinishThreads) void k_argmax_finish(const float* __restrict__ ws_val,
                                                                  const uint32_t* __restrict__ ws_idx, uint32_t nblocks,
                                                                  uint32_t V, uint32_t d, const void* embed,
                                                                  float* x_next, uint32_t* tokens, vsl_ctrl* ctrl) {
    __shared__ float bval[kFinishThreads / 64];
    __shared__ uint32_t bidx[kFinishThreads / 64];
    if (ctrl->done) return;
    const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    float v = -INFINITY;
    uint32_t i = 0xFFFFFFFFu;
    for (uint32_t b = threadIdx.x; b < nblocks; b += kFinishThreads) argmax_merge(v, i, ws_val[b], ws_idx[b]);
    wave_argmax(v, i);
    if (lane == 0) {
        bval[wave] = v;
        bidx[wave] = i;
    }
    __syncthreads();
    if (threadIdx.x < 64) {
        v = threadIdx.x < kFinishThreads / 64 ? bval[threadIdx.x] : -INFINITY;
        i = threadIdx.x < kFinishThreads / 64 ? bidx[threadIdx.x] : 0xFFFFFFFFu;
        wave_argmax(v, i);
        // every logit NaN: greedy_sampling returns 0 (its first element is never beaten)
        if (threadIdx.x == 0) bidx[0] = i == 0xFFFFFFFFu ? 0u : i;
    }
    __syncthreads();
    finish_token<ET>(bidx[0], V, d, embed, x_next, tokens, ctrl);
}

template <int R, int EPI>
uint32_t gemv_blocks(uint32_t N, uint32_t max_blocks) {
    constexpr int RG = (EPI == EPI_SWIGLU) ? R / 2 : R;
    const uint32_t groups = (N + RG - 1) / RG;
    uint32_t blocks = (groups + kWaves - 1) / kWaves;
    if (blocks > max_blocks) blocks = max_blocks;
    return blocks == 0 ? 1 : blocks;
}

template <class WT, int R, int U, int EPI, class ET = WF32>
int launch_gemv(const GemvArgs& a, uint32_t max_blocks, hipStream_t s) {
    const uint32_t blocks = gemv_blocks<R, EPI>(a.N, max_blocks);
    const size_t lds = (size_t)a.K * sizeof(float);
    k_gemv_dec<WT, R, U, EPI, ET><<<blocks, kBlock, lds, s>>>(a);
    HIP_TRY(hipGetLastError());
    return VSL_OK;
}

constexpr uint32_t kMaxK = 16384;  // activation vector held in LDS as fp32 (64 KB)

int check_gemv_shape(uint32_t N, uint32_t K, const char* who) {
    if (N == 0 || K == 0) return vsl_invalid("%s: empty shape", who);
    if (K % 8) return vsl_invalid("%s: K=%u must be a multiple of 8", who, K);
    if (K > kMaxK) return vsl_invalid("%s: K=%u exceeds %u", who, K, kMaxK);
    return VSL_OK;
}

// ---------------------------------------------------------------------------------------------
// flash-decode attention (split-KV, online softmax, in-kernel combine)
// ---------------------------------------------------------------------------------------------
constexpr float kLog2e = 1.4426950408889634f;

template <class KT, int HD, int G>
__global__ __launch_bounds__(kBlock) void k_attn_decode(const float* __restrict__ q, const void* __restrict__ kcache,
                                                        const void* __restrict__ vcache, uint32_t n_q, uint32_t n_kv,
                                                        uint32_t cap, float scale, uint32_t nsplit,
                                                        float* __restrict__ part_o, float* __restrict__ part_ml,
                                                        vsl_ctrl* ctrl) {
    typedef typename KT::T T;
    constexpr int LPP = HD / 8;            // lanes per position (8 elements of 16 bytes... per lane)
    constexpr int SLOTS = 64 / LPP;        // positions per wave per step
    constexpr int NSLOT = kWaves * SLOTS;  // positions per block per step
    __shared__ float s_ml[NSLOT][G][2];
    __shared__ float s_acc[NSLOT][G][HD];

    if (ctrl->done) return;
    const uint32_t pos = ctrl->pos;
    if (pos >= cap) return;
    const uint32_t len = pos + 1;
    const uint32_t kvh = blockIdx.y, split = blockIdx.x;
    uint32_t chunk = (len + nsplit - 1) / nsplit;
    chunk = (chunk + NSLOT - 1) / NSLOT * NSLOT;
    const uint32_t s0 = split * chunk;
    const uint32_t s1 = min(len, s0 + chunk);

    const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const uint32_t slot = lane / LPP, sub = lane % LPP;
    const uint32_t h0 = kvh * G;  // first query head of this KV head (kv_head = head*n_kv/n_q)

    float qv[G][8];
#pragma unroll
    for (int g = 0; g < G; ++g) {
        const float* qp = q + (size_t)(h0 + g) * HD + sub * 8;
        float4 a = *reinterpret_cast<const float4*>(qp);
        float4 b = *reinterpret_cast<const float4*>(qp + 4);
        const float f = scale * kLog2e;
        qv[g][0] = a.x * f; qv[g][1] = a.y * f; qv[g][2] = a.z * f; qv[g][3] = a.w * f;
        qv[g][4] = b.x * f; qv[g][5] = b.y * f; qv[g][6] = b.z * f; qv[g][7] = b.w * f;
    }
    float m[G], l[G], acc[G][8];
#pragma unroll
    for (int g = 0; g < G; ++g) {
        m[g] = -INFINITY;
        l[g] = 0.f;
#pragma unroll
        for (int i = 0; i < 8; ++i) acc[g][i] = 0.f;
    }

    const T* Kb = static_cast<const T*>(kcache) + (size_t)kvh * cap * HD;
    const T* Vb = static_cast<const T*>(vcache) + (size_t)kvh * cap * HD;
    for (uint32_t t = s0 + wave * SLOTS + slot; t < s1; t += NSLOT) {
        float kf[8], vf[8];
        if constexpr (sizeof(T) == 2) {
            uint4 kr = *reinterpret_cast<const uint4*>(Kb + (size_t)t * HD + sub * 8);
            uint4 vr = *reinterpret_cast<const uint4*>(Vb + (size_t)t * HD + sub * 8);
            unpack(kr, WF16(), kf);
            unpack(vr, WF16(), vf);
        } else {
            const float* kp = reinterpret_cast<const float*>(Kb) + (size_t)t * HD + sub * 8;
            const float* vp = reinterpret_cast<const float*>(Vb) + (size_t)t * HD + sub * 8;
            float4 k0 = *reinterpret_cast<const float4*>(kp), k1 = *reinterpret_cast<const float4*>(kp + 4);
            float4 v0 = *reinterpret_cast<const float4*>(vp), v1 = *reinterpret_cast<const float4*>(vp + 4);
            kf[0] = k0.x; kf[1] = k0.y; kf[2] = k0.z; kf[3] = k0.w; kf[4] = k1.x; kf[5] = k1.y; kf[6] = k1.z; kf[7] = k1.w;
            vf[0] = v0.x; vf[1] = v0.y; vf[2] = v0.z; vf[3] = v0.w; vf[4] = v1.x; vf[5] = v1.y; vf[6] = v1.z; vf[7] = v1.w;
        }
#pragma unroll
        for (int g = 0; g < G; ++g) {
            float sc = 0.f;
#pragma unroll
            for (int i = 0; i < 8; ++i) sc = fmaf(qv[g][i], kf[i], sc);
            sc = group_sum<LPP>(sc);
            const float mn = fmaxf(m[g], sc);
            const float corr = exp2f(m[g] - mn);
            const float p = exp2f(sc - mn);
            l[g] = l[g] * corr + p;
#pragma unroll
            for (int i = 0; i < 8; ++i) acc[g][i] = fmaf(p, vf[i], acc[g][i] * corr);
            m[g] = mn;
        }
    }
    // per-slot partials -> LDS -> block combine
    const uint32_t sl = wave * SLOTS + slot;
#pragma unroll
    for (int g = 0; g < G; ++g) {
        if (sub == 0) {
            s_ml[sl][g][0] = m[g];
            s_ml[sl][g][1] = l[g];
        }
#pragma unroll
        for (int i = 0; i < 8; ++i) s_acc[sl][g][sub * 8 + i] = acc[g][i];
    }
    __syncthreads();
    for (uint32_t e = threadIdx.x; e < (uint32_t)(G * HD); e += kBlock) {
        const uint32_t g = e / HD, dd = e % HD;
        float M = -INFINITY;
        for (int s = 0; s < NSLOT; ++s) M = fmaxf(M, s_ml[s][g][0]);
        float L = 0.f, A = 0.f;
        if (M != -INFINITY) {
            for (int s = 0; s < NSLOT; ++s) {
                const float f = exp2f(s_ml[s][g][0] - M);
                L += s_ml[s][g][1] * f;
                A += s_acc[s][g][dd] * f;
            }
        }
        const size_t pidx = (size_t)(h0 + g) * nsplit + split;
        part_o[pidx * HD + dd] = A;
        if (dd == 0) {
            part_ml[pidx * 2 + 0] = M;
            part_ml[pidx * 2 + 1] = L;
        }
    }
}

// Combines the nsplit partials of every query head: out = sum_s A_s 2^(m_s-M) / sum_s l_s 2^(m_s-M).
// One block per head; the split weights are computed once (one thread per split) and the output
// dimensions accumulate over splits with independent loads.
constexpr int kCombineThreads = 128;
constexpr uint32_t kMaxSplits = 1024;
template <int HD>
__global__ __launch_bounds__(kCombineThreads) void k_attn_combine(const float* __restrict__ part_o,
                                                                  const float* __restrict__ part_ml, uint32_t nsplit,
                                                                  float* __restrict__ out, const vsl_ctrl* ctrl) {
    __shared__ float wts[kMaxSplits];
    __shared__ float red[kCombineThreads / 64];
    __shared__ float s_M, s_L;
    if (ctrl->done) return;
    const uint32_t h = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const size_t base = (size_t)h * nsplit;
    float mx = -INFINITY;
    for (uint32_t s = tid; s < nsplit; s += kCombineThreads) {
        const float m = part_ml[(base + s) * 2];
        wts[s] = m;
        mx = fmaxf(mx, m);
    }
    mx = wave_max(mx);
    if (lane == 0) red[wave] = mx;
    __syncthreads();
    if (tid == 0) {
        float M = red[0];
        for (int w = 1; w < kCombineThreads / 64; ++w) M = fmaxf(M, red[w]);
        s_M = M;
    }
    __syncthreads();
    const float M = s_M;
    float lsum = 0.f;
    for (uint32_t s = tid; s < nsplit; s += kCombineThreads) {
        const float m = wts[s];
        const float f = m == -INFINITY ? 0.f : exp2f(m - M);
        wts[s] = f;
        lsum += part_ml[(base + s) * 2 + 1] * f;
    }
    lsum = wave_sum(lsum);
    __syncthreads();
    if (lane == 0) red[wave] = lsum;
    __syncthreads();
    if (tid == 0) {
        float L = 0.f;
        for (int w = 0; w < kCombineThreads / 64; ++w) L += red[w];
        s_L = L;
    }
    __syncthreads();
    const float inv = 1.0f / s_L;
    for (uint32_t dd = tid; dd < (uint32_t)HD; dd += kCombineThreads) {
        float a0 = 0.f, a1 = 0.f, a2 = 0.f, a3 = 0.f;
        uint32_t s = 0;
        for (; s + 4 <= nsplit; s += 4) {
            a0 = fmaf(part_o[(base + s) * HD + dd], wts[s], a0);
            a1 = fmaf(part_o[(base + s + 1) * HD + dd], wts[s + 1], a1);
            a2 = fmaf(part_o[(base + s + 2) * HD + dd], wts[s + 2], a2);
            a3 = fmaf(part_o[(base + s + 3) * HD + dd], wts[s + 3], a3);
        }
        for (; s < nsplit; ++s) a0 = fmaf(part_o[(base + s) * HD + dd], wts[s], a0);
        out[(size_t)h * HD + dd] = ((a0 + a1) + (a2 + a3)) * inv;
    }
}

template <class KT, int HD>
int launch_attn_g(uint32_t G, dim3 grid, hipStream_t s, const float* q, const void* kc, const void* vc, uint32_t n_q,
                  uint32_t n_kv, uint32_t cap, float scale, uint32_t nsplit, float* po, float* pml, float* out,
                  vsl_ctrl* ctrl) {
    switch (G) {
        case 1: k_attn_decode<KT, HD, 1><<<grid, kBlock, 0, s>>>(q, kc, vc, n_q, n_kv, cap, scale, nsplit, po, pml, ctrl); break;
        case 2: k_attn_decode<KT, HD, 2><<<grid, kBlock, 0, s>>>(q, kc, vc, n_q, n_kv, cap, scale, nsplit, po, pml, ctrl); break;
        case 4: k_attn_decode<KT, HD, 4><<<grid, kBlock, 0, s>>>(q, kc, vc, n_q, n_kv, cap, scale, nsplit, po, pml, ctrl); break;
        case 8: k_attn_decode<KT, HD, 8><<<grid, kBlock, 0, s>>>(q, kc, vc, n_q, n_kv, cap, scale, nsplit, po, pml, ctrl); break;
        default: return vsl_unsupported("vsl_attn_decode: GQA ratio %u (supported 1,2,4,8)", G);
    }
    HIP_TRY(hipGetLastError());
    k_attn_combine<HD><<<n_q, kCombineThreads, 0, s>>>(po, pml, nsplit, out, ctrl);
    HIP_TRY(hipGetLastError());
    return VSL_OK;
}

// ---------------------------------------------------------------------------------------------
// samplers on logits in memory (top-k seeded, greedy) -- one block
// ---------------------------------------------------------------------------------------------
constexpr int kSampBlock = 1024;
constexpr int kSampPer = 64;  // values per thread: V <= 65536
constexpr int kMaxTopK = 64;

__device__ __forceinline__ float sample_uniform(uint32_t k0, uint32_t k1, uint64_t step) {
    uint32_t c[4] = {(uint32_t)step, (uint32_t)(step >> 32), 0u, 0u};
    philox4x32_10(c, k0, k1);
    return (float)(c[0] >> 8) * (1.0f / 16777216.0f);
}

// Returns the sampled token in thread 0 (valid for all threads through LDS).
__device__ uint32_t block_sample(const float* __restrict__ logits, uint32_t V, int mode, float temperature,
                                 uint32_t top_k, uint32_t k0, uint32_t k1, uint64_t step) {
    __shared__ float wv[kSampBlock / 64];
    __shared__ uint32_t wi[kSampBlock / 64];
    __shared__ float cand_v[kMaxTopK];
    __shared__ uint32_t cand_i[kMaxTopK];
    __shared__ uint32_t s_tok;
    const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    float vals[kSampPer];
    uint64_t taken = 0;
#pragma unroll
    for (int j = 0; j < kSampPer; ++j) {
        const uint32_t i = tid + (uint32_t)j * kSampBlock;
        vals[j] = i < V ? logits[i] : -INFINITY;
    }
    const bool greedy = (mode == VSL_SAMPLE_GREEDY || mode == VSL_SAMPLE_REFERENCE || temperature <= 0.f);
    uint32_t k = greedy ? 1u : (top_k == 0 || top_k > V ? V : top_k);
    if (k > (uint32_t)kMaxTopK) k = kMaxTopK;
    for (uint32_t it = 0; it < k; ++it) {
        float bv = -INFINITY;
        uint32_t bi = 0xFFFFFFFFu;
#pragma unroll
        for (int j = 0; j < kSampPer; ++j) {
            const uint32_t i = tid + (uint32_t)j * kSampBlock;
            if (i < V && !((taken >> j) & 1ull)) argmax_merge(bv, bi, vals[j], i);
        }
        wave_argmax(bv, bi);
        if (lane == 0) { wv[wave] = bv; wi[wave] = bi; }
        __syncthreads();
        if (tid == 0) {
            float v = wv[0];
            uint32_t i = wi[0];
            for (int w = 1; w < kSampBlock / 64; ++w) argmax_merge(v, i, wv[w], wi[w]);
            if (i == 0xFFFFFFFFu) { i = 0u; v = logits[0]; }
            cand_v[it] = v;
            cand_i[it] = i;
        }
        __syncthreads();
        const uint32_t sel = cand_i[it];
        if (sel % kSampBlock == tid) taken |= 1ull << (sel / kSampBlock);
    }
    if (tid == 0) {
        if (greedy) {
            s_tok = cand_i[0];
        } else {
            // Utils.cpp:151-171 over the k candidates in descending order (ties: lower id first)
            const float mx = cand_v[0];
            float w[kMaxTopK];
            float sum = 0.f;
            for (uint32_t i = 0; i < k; ++i) { w[i] = expf((cand_v[i] - mx) / temperature); sum += w[i]; }
            for (uint32_t i = 0; i < k; ++i) w[i] /= sum;
            const float r = sample_uniform(k0, k1, step);
            float cum = 0.f;
            uint32_t pick = cand_i[0];
            for (uint32_t i = 0; i < k; ++i) {
                cum += w[i];
                if (r < cum) { pick = cand_i[i]; break; }
            }
            s_tok = pick;
        }
    }
    __syncthreads();
    return s_tok;
}

__global__ __launch_bounds__(kSampBlock) void k_sample_logits(const float* logits, uint32_t V, int mode, float T,
                                                              uint32_t top_k, uint32_t k0, uint32_t k1, uint64_t step,
                                                              uint32_t* out) {
    const uint32_t tok = block_sample(logits, V, mode, T, top_k, k0, k1, step);
    if (threadIdx.x == 0) *out = tok;
}

template <class ET>
__global__ __launch_bounds__(kSampBlock) void k_sample_finish(const float* logits, uint32_t V, uint32_t d, int mode,
                                                              float T, uint32_t top_k, uint32_t k0, uint32_t k1,
                                                              const void* embed, float* x_next, uint32_t* tokens,
                                                              vsl_ctrl* ctrl) {
    if (ctrl->done) return;
    const uint32_t tok = block_sample(logits, V, mode, T, top_k, k0, k1, ctrl->step);
    finish_token<ET>(tok, V, d, embed, x_next, tokens, ctrl);
}

// ---------------------------------------------------------------------------------------------
// embedding gather and row RMSNorm (prefill side)
// ---------------------------------------------------------------------------------------------
template <class ET>
__global__ void k_embed(const void* table, uint32_t vocab, uint32_t d, const uint32_t* ids, uint32_t n, float* out) {
    const uint32_t t = blockIdx.x;
    if (t >= n) return;
    uint32_t id = ids[t];
    id = id < vocab ? id : vocab - 1;  // embedding_lookup.comp:32
    const typename ET::T* e = static_cast<const typename ET::T*>(table) + (size_t)id * d;
    for (uint32_t i = threadIdx.x; i < d; i += blockDim.x) out[(size_t)t * d + i] = to_f32(e[i]);
}

template <typename OT, bool X2>
__global__ __launch_bounds__(kBlock) void k_rmsnorm_rows(const float* x, const float* gamma, uint32_t rows, uint32_t d,
                                                         float eps, OT* out) {
    __shared__ float red[kWaves];
    const float* xr = x + (size_t)blockIdx.x * d;
    float ss = 0.f;
    for (uint32_t i = threadIdx.x; i < d; i += kBlock) ss += xr[i] * xr[i];
    ss = wave_sum(ss);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = ss;
    __syncthreads();
    float tot = 0.f;
    for (int w = 0; w < kWaves; ++w) tot += red[w];
    const float inv = 1.0f / sqrtf(tot / (float)d + eps);
    for (uint32_t i = threadIdx.x; i < d; i += kBlock) {
        const float v = xr[i] * inv * (gamma ? gamma[i] : 1.0f);
        if constexpr (X2) {
            const vsl_half hi = (vsl_half)v;
            out[(size_t)blockIdx.x * d + i] = hi;
            out[(size_t)rows * d + (size_t)blockIdx.x * d + i] = (vsl_half)(v - (float)hi);
        } else {
            store_elem(out + (size_t)blockIdx.x * d + i, v);
        }
    }
}

// ---------------------------------------------------------------------------------------------
// GEMV sweep for B > 1: X staged per K-chunk in LDS (fp32), R rows per wave, B columns.
// ---------------------------------------------------------------------------------------------
template <class WT, int B, typename XT, typename YT>
__global__ __launch_bounds__(kBlock) void k_gemv_multi(const void* Wv, uint32_t N, uint32_t K, const XT* X, YT* Y) {
    constexpr int VEC = WT::kVec;
    constexpr uint32_t KC = 64 * VEC;  // one 16-byte load per lane per row per chunk
    constexpr int R = 2;
    __shared__ float xs[KC * B];
    typedef typename WT::T T;
    const T* W = static_cast<const T*>(Wv);
    const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const uint32_t row0 = (blockIdx.x * kWaves + wave) * R;
    float acc[R][B];
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int b = 0; b < B; ++b) acc[r][b] = 0.f;
    for (uint32_t k0 = 0; k0 < K; k0 += KC) {
        __syncthreads();
        for (uint32_t e = threadIdx.x; e < KC * B; e += kBlock) {
            const uint32_t kk = k0 + e / B;
            xs[e] = kk < K ? to_f32(X[(size_t)kk * B + (e % B)]) : 0.f;
        }
        __syncthreads();
        const uint32_t kk = k0 + lane * VEC;
        if (kk < K) {
#pragma unroll
            for (int r = 0; r < R; ++r) {
                const uint32_t row = row0 + r;
                if (row >= N) continue;
                float wf[VEC];
                unpack(load16<true>(W + (size_t)row * K + kk), WT(), wf);
#pragma unroll
                for (int i = 0; i < VEC; ++i)
#pragma unroll
                    for (int b = 0; b < B; ++b) acc[r][b] = fmaf(wf[i], xs[(lane * VEC + i) * B + b], acc[r][b]);
            }
        }
    }
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const uint32_t row = row0 + r;
#pragma unroll
        for (int b = 0; b < B; ++b) {
            const float v = wave_sum(acc[r][b]);
            if (lane == 0 && row < N) store_elem(Y + (size_t)row * B + b, v);
        }
    }
}

template <class WT, typename XT, typename YT>
int launch_gemv_multi(const void* W, uint32_t N, uint32_t K, const void* X, uint32_t B, void* Y, hipStream_t s) {
    const uint32_t blocks = (N + kWaves * 2 - 1) / (kWaves * 2);
    const XT* x = static_cast<const XT*>(X);
    YT* y = static_cast<YT*>(Y);
    switch (B) {
#define VSL_CASE(b) case b: k_gemv_multi<WT, b, XT, YT><<<blocks, kBlock, 0, s>>>(W, N, K, x, y); break;
        VSL_CASE(2) VSL_CASE(3) VSL_CASE(4) VSL_CASE(5) VSL_CASE(6) VSL_CASE(7) VSL_CASE(8) VSL_CASE(9)
        VSL_CASE(10) VSL_CASE(11) VSL_CASE(12) VSL_CASE(13) VSL_CASE(14) VSL_CASE(15) VSL_CASE(16)
#undef VSL_CASE
        default: return vsl_invalid("vsl_gemv: B=%u out of range", B);
    }
    HIP_TRY(hipGetLastError());
    return VSL_OK;
}

// fp16 -> fp32 staging of a single activation column (sweep B=1 with f16 X)
__global__ void k_h2f(const vsl_half* x, float* y, uint32_t n) {
    for (uint32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x) y[i] = (float)x[i];
}

}  // namespace

// =============================================================================================
// C ABI
// =============================================================================================
extern "C" int vsl_embed(const void* table, int dtype, uint32_t vocab, uint32_t d, const uint32_t* ids_dev, uint32_t n,
                         float* out, void* stream) {
    if (!table || !ids_dev || !out || vocab == 0 || d == 0) return vsl_invalid("vsl_embed: bad arguments");
    if (n == 0) return VSL_OK;
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (dtype == VSL_DT_F16)
        k_embed<WF16><<<n, kBlock, 0, s>>>(table, vocab, d, ids_dev, n, out);
    else if (dtype == VSL_DT_F32)
        k_embed<WF32><<<n, kBlock, 0, s>>>(table, vocab, d, ids_dev, n, out);
    else
        return vsl_unsupported("vsl_embed: dtype %d", dtype);
    HIP_TRY(hipGetLastError());
    return VSL_OK;
}

extern "C" int vsl_rmsnorm(const float* x, const float* gamma, uint32_t rows, uint32_t d, float eps, void* out,
                           int out_dtype, void* stream) {
    if (!x || !out || d == 0) return vsl_invalid("vsl_rmsnorm: bad arguments");
    if (rows == 0) return VSL_OK;
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (out_dtype == VSL_DT_F16)
        k_rmsnorm_rows<vsl_half, false><<<rows, kBlock, 0, s>>>(x, gamma, rows, d, eps, static_cast<vsl_half*>(out));
    else if (out_dtype == VSL_DT_F16X2)
        k_rmsnorm_rows<vsl_half, true><<<rows, kBlock, 0, s>>>(x, gamma, rows, d, eps, static_cast<vsl_half*>(out));
    else if (out_dtype == VSL_DT_F32)
        k_rmsnorm_rows<float, false><<<rows, kBlock, 0, s>>>(x, gamma, rows, d, eps, static_cast<float*>(out));
    else
        return vsl_unsupported("vsl_rmsnorm: dtype %d", out_dtype);
    HIP_TRY(hipGetLastError());
    return VSL_OK;
}

extern "C" int vsl_gemv(const void* W, int wdtype, uint32_t N, uint32_t K, const void* X, int xdtype, uint32_t B,
                        void* Y, int ydtype, void* stream) {
    if (!W || !X || !Y) return vsl_invalid("vsl_gemv: null pointer");
    if (int rc = check_gemv_shape(N, K, "vsl_gemv")) return rc;
    if (B < 1 || B > 16) return vsl_invalid("vsl_gemv: B=%u must be in [1,16]", B);
    if ((wdtype != VSL_DT_F16 && wdtype != VSL_DT_F32) || (xdtype != VSL_DT_F16 && xdtype != VSL_DT_F32) ||
        (ydtype != VSL_DT_F16 && ydtype != VSL_DT_F32))
        return vsl_unsupported("vsl_gemv: dtype combination %d/%d/%d", wdtype, xdtype, ydtype);
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (B == 1) {
        if (xdtype == VSL_DT_F16) return vsl_unsupported("vsl_gemv: B=1 expects fp32 X (use the f16 path via B>1)");
        GemvArgs a{};
        a.W = W;
        a.N = N;
        a.K = K;
        a.x = static_cast<const float*>(X);
        a.y = static_cast<float*>(Y);
        if (wdtype == VSL_DT_F16)
            return ydtype == VSL_DT_F16 ? launch_gemv<WF16, 2, 8, EPI_STORE_F16>(a, 1u << 20, s)
                                        : launch_gemv<WF16, 2, 8, EPI_STORE>(a, 1u << 20, s);
        return ydtype == VSL_DT_F16 ? launch_gemv<WF32, 2, 8, EPI_STORE_F16>(a, 1u << 20, s)
                                    : launch_gemv<WF32, 2, 8, EPI_STORE>(a, 1u << 20, s);
    }
#define VSL_DISPATCH_XY(WT)                                                                                 \
    if (xdtype == VSL_DT_F16 && ydtype == VSL_DT_F16) return launch_gemv_multi<WT, vsl_half, vsl_half>(W, N, K, X, B, Y, s); \
    if (xdtype == VSL_DT_F16 && ydtype == VSL_DT_F32) return launch_gemv_multi<WT, vsl_half, float>(W, N, K, X, B, Y, s);    \
    if (xdtype == VSL_DT_F32 && ydtype == VSL_DT_F16) return launch_gemv_multi<WT, float, vsl_half>(W, N, K, X, B, Y, s);    \
    return launch_gemv_multi<WT, float, float>(W, N, K, X, B, Y, s);
    if (wdtype == VSL_DT_F16) {
        VSL_DISPATCH_XY(WF16)
    }
    VSL_DISPATCH_XY(WF32)
#undef VSL_DISPATCH_XY
}

extern "C" int vsl_qkv_rope_append(const float* x, const float* gamma, float eps, const void* Wqkv, int wdtype,
                                   uint32_t d, uint32_t n_q, uint32_t n_kv, uint32_t hd, const float* rope_cos,
                                   const float* rope_sin, void* kcache, void* vcache, int kv_dtype, uint32_t cap,
                                   float* q_out, vsl_ctrl* ctrl, void* stream) {
    if (!x || !Wqkv || !rope_cos || !rope_sin || !kcache || !vcache || !q_out || !ctrl)
        return vsl_invalid("vsl_qkv_rope_append: null pointer");
    if (hd % 8 || hd == 0 || n_q == 0 || n_kv == 0) return vsl_invalid("vsl_qkv_rope_append: bad head shape");
    const uint32_t N = (n_q + 2 * n_kv) * hd;
    if (int rc = check_gemv_shape(N, d, "vsl_qkv_rope_append")) return rc;
    GemvArgs a{};
    a.W = Wqkv; a.N = N; a.K = d; a.x = x; a.gamma = gamma; a.eps = eps;
    a.n_q = n_q; a.n_kv = n_kv; a.hd = hd; a.cap = cap; a.rope_cos = rope_cos; a.rope_sin = rope_sin;
    a.kc = kcache; a.vc = vcache; a.q_out = q_out; a.ctrl = ctrl;
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (wdtype == VSL_DT_F16) {
        if (kv_dtype == VSL_DT_F16) return launch_gemv<WF16, 2, 8, EPI_QKV, WF16>(a, 1u << 20, s);
        return launch_gemv<WF16, 2, 8, EPI_QKV, WF32>(a, 1u << 20, s);
    }
    if (wdtype == VSL_DT_F32) {
        if (kv_dtype == VSL_DT_F16) return launch_gemv<WF32, 2, 8, EPI_QKV, WF16>(a, 1u << 20, s);
        return launch_gemv<WF32, 2, 8, EPI_QKV, WF32>(a, 1u << 20, s);
    }
    return vsl_unsupported("vsl_qkv_rope_append: dtype %d", wdtype);
}

extern "C" int vsl_attn_decode(const float* q, const void* kcache, const void* vcache, int kv_dtype, uint32_t n_q,
                               uint32_t n_kv, uint32_t hd, uint32_t cap, float scale, uint32_t nsplit, float* part_o,
                               float* part_ml, float* out, vsl_ctrl* ctrl, void* stream) {
    if (!q || !kcache || !vcache || !part_o || !part_ml || !out || !ctrl)
        return vsl_invalid("vsl_attn_decode: null pointer");
    if (n_kv == 0 || n_q % n_kv) return vsl_invalid("vsl_attn_decode: n_q=%u not a multiple of n_kv=%u", n_q, n_kv);
    if (nsplit == 0 || nsplit > kMaxSplits) return vsl_invalid("vsl_attn_decode: nsplit=%u (1..%u)", nsplit, kMaxSplits);
    const uint32_t G = n_q / n_kv;
    dim3 grid(nsplit, n_kv);
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (kv_dtype == VSL_DT_F16) {
        if (hd == 128) return launch_attn_g<WF16, 128>(G, grid, s, q, kcache, vcache, n_q, n_kv, cap, scale, nsplit, part_o, part_ml, out, ctrl);
        if (hd == 64) return launch_attn_g<WF16, 64>(G, grid, s, q, kcache, vcache, n_q, n_kv, cap, scale, nsplit, part_o, part_ml, out, ctrl);
    } else if (kv_dtype == VSL_DT_F32) {
        if (hd == 128) return launch_attn_g<WF32, 128>(G, grid, s, q, kcache, vcache, n_q, n_kv, cap, scale, nsplit, part_o, part_ml, out, ctrl);
        if (hd == 64) return launch_attn_g<WF32, 64>(G, grid, s, q, kcache, vcache, n_q, n_kv, cap, scale, nsplit, part_o, part_ml, out, ctrl);
    }
    return vsl_unsupported("vsl_attn_decode: head_dim %u / kv dtype %d (supported 64,128 / f16,f32)", hd, kv_dtype);
}

extern "C" int vsl_gemv_residual(const void* W, int wdtype, uint32_t N, uint32_t K, const float* x, float* resid,
                                 vsl_ctrl* ctrl, void* stream) {
    if (!W || !x || !resid) return vsl_invalid("vsl_gemv_residual: null pointer");
    if (int rc = check_gemv_shape(N, K, "vsl_gemv_residual")) return rc;
    GemvArgs a{};
    a.W = W; a.N = N; a.K = K; a.x = x; a.y = resid; a.ctrl = ctrl;
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (wdtype == VSL_DT_F16) return launch_gemv<WF16, 2, 8, EPI_RESID>(a, 1u << 20, s);
    if (wdtype == VSL_DT_F32) return launch_gemv<WF32, 2, 8, EPI_RESID>(a, 1u << 20, s);
    return vsl_unsupported("vsl_gemv_residual: dtype %d", wdtype);
}

extern "C" int vsl_norm_swiglu(const float* x, const float* gamma, float eps, const void* Wgu, int wdtype, uint32_t d,
                               uint32_t F, float* h_out, vsl_ctrl* ctrl, void* stream) {
    if (!x || !Wgu || !h_out) return vsl_invalid("vsl_norm_swiglu: null pointer");
    if (int rc = check_gemv_shape(F, d, "vsl_norm_swiglu")) return rc;
    GemvArgs a{};
    a.W = Wgu; a.N = F; a.K = d; a.x = x; a.gamma = gamma; a.eps = eps; a.y = h_out; a.ctrl = ctrl;
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (wdtype == VSL_DT_F16) return launch_gemv<WF16, 4, 4, EPI_SWIGLU>(a, 1u << 20, s);
    if (wdtype == VSL_DT_F32) return launch_gemv<WF32, 4, 4, EPI_SWIGLU>(a, 1u << 20, s);
    return vsl_unsupported("vsl_norm_swiglu: dtype %d", wdtype);
}

extern "C" uint32_t vsl_lm_head_ws_blocks(void) { return kMaxLmBlocks; }

extern "C" int vsl_lm_head_sample(const float* gamma, float eps, const void* W, int wdtype, uint32_t V, uint32_t d,
                                  float* x, const void* embed, int embed_dtype, float* logits, vsl_sampler sampler,
                                  float* ws_val, uint32_t* ws_idx, uint32_t* tokens, vsl_ctrl* ctrl, void* stream) {
    if (!W || !x || !embed || !logits || !ws_val || !ws_idx || !tokens || !ctrl)
        return vsl_invalid("vsl_lm_head_sample: null pointer");
    if (int rc = check_gemv_shape(V, d, "vsl_lm_head_sample")) return rc;
    if (embed_dtype != VSL_DT_F16 && embed_dtype != VSL_DT_F32) return vsl_unsupported("embed dtype %d", embed_dtype);
    if (wdtype != VSL_DT_F16 && wdtype != VSL_DT_F32) return vsl_unsupported("vsl_lm_head_sample: dtype %d", wdtype);
    hipStream_t s = static_cast<hipStream_t>(stream);
    const bool fused = sampler.mode == VSL_SAMPLE_GREEDY || sampler.mode == VSL_SAMPLE_REFERENCE ||
                       sampler.temperature <= 0.f;
    GemvArgs a{};
    a.W = W; a.N = V; a.K = d; a.x = x; a.gamma = gamma; a.eps = eps; a.y = logits;
    a.ws_val = ws_val; a.ws_idx = ws_idx; a.tokens = tokens; a.embed = embed; a.x_next = x;
    a.ctrl = ctrl;
    if (fused) {
        int rc = wdtype == VSL_DT_F16 ? launch_gemv<WF16, 2, 8, EPI_ARGMAX>(a, kMaxLmBlocks, s)
                                      : launch_gemv<WF32, 2, 8, EPI_ARGMAX>(a, kMaxLmBlocks, s);
        if (rc) return rc;
        const uint32_t nb = gemv_blocks<2, EPI_ARGMAX>(V, kMaxLmBlocks);
        if (embed_dtype == VSL_DT_F16)
            k_argmax_finish<WF16><<<1, kFinishThreads, 0, s>>>(ws_val, ws_idx, nb, V, d, embed, x, tokens, ctrl);
        else
            k_argmax_finish<WF32><<<1, kFinishThreads, 0, s>>>(ws_val, ws_idx, nb, V, d, embed, x, tokens, ctrl);
        HIP_TRY(hipGetLastError());
        return VSL_OK;
    }
    if (sampler.mode != VSL_SAMPLE_TOPK_SEEDED) return vsl_invalid("vsl_lm_head_sample: sampler mode %d", sampler.mode);
    if (V > (uint32_t)(kSampBlock * kSampPer)) return vsl_unsupported("top-k sampling supports V <= %d", kSampBlock * kSampPer);
    // logits only (EPI_STORE with the norm prologue), then the sampling kernel
    int rc = wdtype == VSL_DT_F16 ? launch_gemv<WF16, 2, 8, EPI_STORE>(a, 1u << 20, s)
                                  : launch_gemv<WF32, 2, 8, EPI_STORE>(a, 1u << 20, s);
    if (rc) return rc;
    const uint64_t key = vsl_derive_key(sampler.seed, "sampler");
    if (embed_dtype == VSL_DT_F16)
        k_sample_finish<WF16><<<1, kSampBlock, 0, s>>>(logits, V, d, sampler.mode, sampler.temperature, sampler.top_k,
                                                       (uint32_t)key, (uint32_t)(key >> 32), embed, x, tokens, ctrl);
    else
        k_sample_finish<WF32><<<1, kSampBlock, 0, s>>>(logits, V, d, sampler.mode, sampler.temperature, sampler.top_k,
                                                       (uint32_t)key, (uint32_t)(key >> 32), embed, x, tokens, ctrl);
    HIP_TRY(hipGetLastError());
    return VSL_OK;
}

extern "C" int vsl_sample_logits(const float* logits, uint32_t V, vsl_sampler sampler, uint64_t step, uint32_t* out,
                                 void* stream) {
    if (!logits || !out || V == 0) return vsl_invalid("vsl_sample_logits: bad arguments");
    if (V > (uint32_t)(kSampBlock * kSampPer)) return vsl_unsupported("sampling supports V <= %d", kSampBlock * kSampPer);
    if (sampler.mode < 0 || sampler.mode > 2) return vsl_invalid("vsl_sample_logits: mode %d", sampler.mode);
    const uint64_t key = vsl_derive_key(sampler.seed, "sampler");
    k_sample_logits<<<1, kSampBlock, 0, static_cast<hipStream_t>(stream)>>>(
        logits, V, sampler.mode, sampler.temperature, sampler.top_k, (uint32_t)key, (uint32_t)(key >> 32), step, out);
    HIP_TRY(hipGetLastError());
    return VSL_OK;
}
