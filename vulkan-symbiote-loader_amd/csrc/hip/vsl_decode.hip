// vsl_decode.hip -- bs=1 decode kernels for gfx950.
//
// Every decode-step GEMV is HBM-bound (1 flop/byte): the kernels stream each weight row once with
// 16-byte loads, keep the (normalised) activation vector in LDS as fp32, reduce across the 64-lane
// wavefront with butterfly shuffles, and fuse the neighbouring elementwise op into the epilogue:
//   k_gemv_dec<EPI_QKV>    RMSNorm -> [Wq;Wk;Wv] -> RoPE -> q + KV-cache append
//   k_gemv_dec<EPI_RESID>  W_o / W_down -> residual add
//   k_gemv_dec<EPI_SWIGLU> RMSNorm -> [Wgate;Wup] -> silu(g)*u
//   k_gemv_dec<EPI_ARGMAX> final RMSNorm -> W_out -> logits + fused greedy argmax + next embedding
// k_attn_decode is a split-KV flash-decode kernel whose partials k_attn_combine merges.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <mutex>
#include <type_traits>

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
    const vsl_half* xh;  // when set, the activation vector is fp16 (8-byte aligned) and x is unused
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
// Barrier for LDS traffic only: waits for this wave's LDS operations, not for its outstanding
// global loads (the weight stream keeps flowing across it).
__device__ __forceinline__ void lds_barrier() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// Float4 slot of the activation vector's float4 q in LDS for the block-quantized tiles. A lane reads
// kVec / 4 consecutive float4s per weight load (lanes kVec floats apart), so in the plain layout the
// lanes of one LDS pass hit the same banks 4-fold (Q8) or 8-fold (Q4). XOR-ing the slot within its
// aligned group of eight with bits 3-5 ^ 4-6 of q spreads every such pass, and the staging stores of
// consecutive float4s, over distinct banks for 32 or 64 banks of 4 bytes; it only permutes slots
// within aligned groups of 8 float4s, so the vector fits in K rounded up to 32 floats. (fp16 tiles,
// 2-fold in the plain layout, keep it: with the slot XORs the 8B decode's down and O projections took
// 19.80 / 7.16 us against 19.64 / 7.04, kernel-trace medians.)
__device__ __forceinline__ uint32_t xs_slot(uint32_t q) { return q ^ (((q >> 3) ^ (q >> 4)) & 7u); }
template <class WT>
__device__ __host__ constexpr bool xs_swizzled() { return WT::kQuant; }
__device__ __host__ __forceinline__ constexpr uint32_t xs_floats(uint32_t K) { return (K + 31u) & ~31u; }

// The block's activation slice lives in registers between its loads and the LDS store, so that
// the loads can be issued ahead of the first weight tile (vector loads complete in issue order:
// waiting for the activations then never waits for the weights behind them).
template <int WAVES, int XPT>
struct XStage {
    static constexpr uint32_t NT = WAVES * 64;  // XPT float4 per thread: K <= XPT * NT * 4
    float4 xr[XPT];
    float4 gr[XPT];

    // Branch-free, with indexes past K clamped to 0: the waits that later consume these registers
    // then count exactly the loads issued after them.
    // (the gains only when there is a norm; these loads all precede the first weight tile, so a
    // uniform branch here changes no wait of the weight pipeline)
    __device__ __forceinline__ void load(const float* __restrict__ x, const vsl_half* __restrict__ xh,
                                         const float* __restrict__ gamma, uint32_t K) {
        const uint32_t tid = threadIdx.x;
        if (xh) {  // fp16 activations (a uniform branch ahead of every weight load)
#pragma unroll
            for (int j = 0; j < XPT; ++j) {
                const uint32_t i = (j * NT + tid) * 4;
                const uint32_t ic = i < K ? i : 0;
                const uint2 hv = *reinterpret_cast<const uint2*>(xh + ic);
                const half2v a = __builtin_bit_cast(half2v, hv.x), b = __builtin_bit_cast(half2v, hv.y);
                xr[j] = make_float4((float)a[0], (float)a[1], (float)b[0], (float)b[1]);
            }
        } else {
#pragma unroll
            for (int j = 0; j < XPT; ++j) {
                const uint32_t i = (j * NT + tid) * 4;
                const uint32_t ic = i < K ? i : 0;
                xr[j] = *reinterpret_cast<const float4*>(x + ic);
            }
        }
        if (gamma) {
#pragma unroll
            for (int j = 0; j < XPT; ++j) {
                const uint32_t i = (j * NT + tid) * 4;
                const uint32_t ic = i < K ? i : 0;
                gr[j] = *reinterpret_cast<const float4*>(gamma + ic);
            }
        } else {
#pragma unroll
            for (int j = 0; j < XPT; ++j) gr[j] = make_float4(1.f, 1.f, 1.f, 1.f);
        }
    }
    // RMS-normalise (rms_norm.comp:24-34) when gamma is given, and store to LDS as fp32 (with SWZ,
    // float4 q at slot xs_slot(q)); with BSUM (K % 32 == 0) also the sum of every 32-value block, at
    // xs[K + i / 32]
    template <bool SWZ, bool BSUM>
    __device__ __forceinline__ void store(const float* __restrict__ gamma, float eps, uint32_t K, float* __restrict__ xs,
                                          float* red) {
        const uint32_t tid = threadIdx.x;
        // Read every staged register here, on every path: the branches below would otherwise leave
        // some loads pending, and the loop's first weight issue would wait on them.
#pragma unroll
        for (int j = 0; j < XPT; ++j) {
            asm volatile("" ::"v"(xr[j].x), "v"(xr[j].y), "v"(xr[j].z), "v"(xr[j].w));
            asm volatile("" ::"v"(gr[j].x), "v"(gr[j].y), "v"(gr[j].z), "v"(gr[j].w));
        }
        float inv = 1.f;
        if (gamma) {
            float ss = 0.f;
#pragma unroll
            for (int j = 0; j < XPT; ++j) {
                const uint32_t i = (j * NT + tid) * 4;
                if (j * NT * 4 < K && i < K) {
                    const float4 v = xr[j];
                    ss += v.x * v.x + v.y * v.y + v.z * v.z + v.w * v.w;
                }
            }
            ss = wave_sum_dpp(ss);
            if ((tid & 63) == 0) red[tid >> 6] = ss;
            lds_barrier();
            float tot = 0.f;
#pragma unroll
            for (int w = 0; w < WAVES; ++w) tot += red[w];
            inv = 1.0f / sqrtf(tot / (float)K + eps);
        }
#pragma unroll
        for (int j = 0; j < XPT; ++j) {
            const uint32_t i = (j * NT + tid) * 4;
            if (j * NT * 4 < K) {  // uniform: the block sums below take whole lane groups
                const bool in = i < K;
                float4 v = xr[j];
                if (gamma) {
                    const float4 g = gr[j];
                    v.x = v.x * inv * g.x;
                    v.y = v.y * inv * g.y;
                    v.z = v.z * inv * g.z;
                    v.w = v.w * inv * g.w;
                }
                if (in) reinterpret_cast<float4*>(xs)[SWZ ? xs_slot(i / 4) : i / 4] = v;
                if constexpr (BSUM) {
                    // a 32-value block is the float4s of 8 adjacent lanes
                    float bs = in ? (v.x + v.y) + (v.z + v.w) : 0.f;
                    bs = group_sum_dpp<8>(bs);
                    if (in && (tid & 7) == 0) xs[K + i / 32] = bs;
                }
            }
        }
        lds_barrier();
    }
};

// The kVec activations of columns kk .. kk + kVec - 1 (kk a multiple of kVec). Quantized tiles: the
// float4s q0 .. q0 + F - 1 of one aligned group of eight, at slots xs_slot(q0) ^ j = (q0 ^ g) ^ j, with
// g = xs_slot(q0) ^ q0 the lane's constant (bits 0-6 of q0 = kk / 4 come from lane * F alone, the
// tile's column base being a multiple of 512 floats).
template <class WT>
__device__ __forceinline__ void load_x(const float* xs, uint32_t kk, float* xv, uint32_t g) {
    const float4* x4 = reinterpret_cast<const float4*>(xs);
    const uint32_t p0 = xs_swizzled<WT>() ? (kk >> 2) ^ g : kk >> 2;
#pragma unroll
    for (int j = 0; j < WT::kVec / 4; ++j) {
        const float4 a = x4[xs_swizzled<WT>() ? p0 ^ (uint32_t)j : p0 + j];
        xv[4 * j] = a.x; xv[4 * j + 1] = a.y; xv[4 * j + 2] = a.z; xv[4 * j + 3] = a.w;
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
// Work unit: a row group (R weight rows; EPI_SWIGLU: R/2 gate rows + the matching up rows) split
// into K-chunks of U x 64 lanes x 16 bytes. A wave walks its tiles (group, chunk) with two register
// buffers: tile t+1 is requested before tile t is consumed, so every wave keeps one tile in
// flight at all times, including across its row-group boundaries. Operands the epilogue reads
// from memory (residual rows, RoPE angles) are requested together with each tile.
template <class WT, int R, int U, int EPI, class ET, int WAVES, int XPT>
__global__ __launch_bounds__(WAVES * 64) void k_gemv_dec(GemvArgs a) {
    __shared__ float red[WAVES];
    __shared__ float bval[WAVES];
    __shared__ uint32_t bidx[WAVES];
    extern __shared__ float xs[];

    constexpr int VEC = WT::kVec;
    constexpr bool QW = WT::kQuant;  // block-quantized pack: values, then scales (and offsets)
    constexpr uint32_t SPAN = 64 * VEC;
    constexpr uint32_t CHUNK = SPAN * U;
    constexpr int RG = (EPI == EPI_SWIGLU) ? R / 2 : R;  // logical rows per group
    static_assert(EPI != EPI_SWIGLU || R % 2 == 0, "SwiGLU groups pair gate and up rows");
    static_assert(EPI != EPI_QKV || R % 2 == 0, "QKV groups hold whole RoPE pairs");
    static_assert(!QW || VEC <= 32, "a lane's quantized values lie in one 32-value block");
    const char* __restrict__ W = static_cast<const char*>(a.W);
    // quantized packs: the scale (and offset) of the 32-value block of element e is plane[e / 32]
    const uint64_t w_rows = EPI == EPI_SWIGLU ? 2ull * a.N : a.N;
    const float* __restrict__ Qs = QW ? reinterpret_cast<const float*>(W + qpack_scales_off(WT::kBits, w_rows, a.K)) : nullptr;
    const float* __restrict__ Qm = WT::kMin ? reinterpret_cast<const float*>(W + qpack_mins_off(WT::kBits, w_rows, a.K)) : nullptr;
    const uint32_t lane = threadIdx.x & 63;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform
    static_assert(!xs_swizzled<WT>() || SPAN % 512 == 0, "the activation slot constant needs 512-float column bases");
    const uint32_t xg = xs_slot(lane * (VEC / 4)) ^ (lane * (VEC / 4));  // load_x's slot constant
    const uint32_t n_groups = (a.N + RG - 1) / RG;
    const uint32_t stride = gridDim.x * WAVES;
    const uint32_t g0 = blockIdx.x * WAVES + wave;
    const uint32_t cpg = (a.K + CHUNK - 1) / CHUNK;  // chunks per group
    const uint32_t n_tiles = g0 < n_groups ? ((n_groups - 1 - g0) / stride + 1) * cpg : 0;

    uint32_t pos = 0;

    auto group_rows = [&](uint32_t g, uint32_t* rows, bool* ok) {
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
    };
    // weights of tile t (with the block scales and offsets of a quantized pack)
    auto issue_w = [&](uint4 (&w)[R][U], float (&qs)[R][U], float (&qm)[R][U], uint32_t t) {
        const uint32_t gi = t / cpg, c = t - gi * cpg;
        const uint32_t k0 = c * CHUNK;
        uint32_t rows[R];
        bool ok[R];
        group_rows(g0 + gi * stride, rows, ok);
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const uint32_t kk = k0 + u * SPAN + lane * VEC;
#pragma unroll
            for (int r = 0; r < R; ++r) {
                // Out-of-range rows and columns load element 0 of the matrix instead: no branch
                // or select touches a tile between its loads and its use (columns past K are
                // skipped in consume, rows past N never reach an output).
                const bool in = ok[r] && kk < a.K;
                const uint64_t e = in ? (uint64_t)rows[r] * a.K + kk : 0;
                w[r][u] = load16<true>(W + wt_bytes<WT>(e));
                if constexpr (QW) qs[r][u] = Qs[e / 32];
                if constexpr (WT::kMin) qm[r][u] = Qm[e / 32];
            }
        }
    };
    // operands the epilogue reads from memory
    // (requested with every tile, so that no branch separates a tile's loads from their waits)
    auto issue_pf = [&](float (&pf)[R], uint32_t t) {
        const uint32_t gi = t / cpg;
        uint32_t rows[R];
        bool ok[R];
        group_rows(g0 + gi * stride, rows, ok);
        // addresses are clamped in range; rows past N are never stored
        if constexpr (EPI == EPI_RESID) {
#pragma unroll
            for (int r = 0; r < R; ++r) pf[r] = a.y[ok[r] ? rows[r] : 0];
        } else if constexpr (EPI == EPI_QKV) {
            const uint32_t half = a.hd >> 1;
#pragma unroll
            for (int r = 0; r < R; r += 2) {
                const size_t ti = (size_t)pos * half + ((rows[r] % a.hd) >> 1);  // pos < cap here
                pf[r] = a.rope_cos[ti];
                pf[r + 1] = a.rope_sin[ti];
            }
        }
    };
    auto issue = [&](uint4 (&w)[R][U], float (&qs)[R][U], float (&qm)[R][U], float (&pf)[R], uint32_t t) {
        issue_w(w, qs, qm, t);
        issue_pf(pf, t);
    };

    float acc[R];
#pragma unroll
    for (int r = 0; r < R; ++r) acc[r] = 0.f;
    float best_v = -INFINITY;
    uint32_t best_i = 0xFFFFFFFFu;

    auto epilogue = [&](uint32_t g, const float (&pf)[R]) {
        uint32_t rows[R];
        bool ok[R];
        group_rows(g, rows, ok);
#pragma unroll
        for (int r = 0; r < R; ++r) acc[r] = wave_sum_dpp(acc[r]);
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
                    if (ok[r]) a.y[rows[r]] = pf[r] + acc[r];
            }
        } else if constexpr (EPI == EPI_SWIGLU) {
            if (lane == 0) {
#pragma unroll
                for (int r = 0; r < RG; ++r)
                    if (ok[r]) a.y[rows[r]] = silu(acc[r]) * acc[r + RG];
            }
        } else if constexpr (EPI == EPI_QKV) {
            if (lane == 0) {
                const uint32_t qrows = a.n_q * a.hd, krows = a.n_kv * a.hd;
#pragma unroll
                for (int r = 0; r < R; r += 2) {
                    if (!ok[r]) continue;
                    const uint32_t row = rows[r];
                    // RoPE on q and k rows (adjacent pair row, row+1); v rows pass through
                    const bool rot = row < qrows + krows;
                    const float c = rot ? pf[r] : 1.f, sn = rot ? pf[r + 1] : 0.f;
                    const float v0 = acc[r] * c - acc[r + 1] * sn;
                    const float v1 = acc[r] * sn + acc[r + 1] * c;
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
#pragma unroll
        for (int r = 0; r < R; ++r) acc[r] = 0.f;
    };
    // Every register of a tile is read on every path (columns past K are zeroed by selects, not
    // skipped by branches), so no path leaves a load pending into the next issue of its buffer.
    auto consume = [&](const uint4 (&w)[R][U], const float (&qs)[R][U], const float (&qm)[R][U], const float (&pf)[R],
                       uint32_t t) {
        const uint32_t gi = t / cpg, c = t - gi * cpg;
        const uint32_t k0 = c * CHUNK;
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const uint32_t kk = k0 + u * SPAN + lane * VEC;
            const bool in = kk < a.K;
            float xv[VEC];
            load_x<WT>(xs, in ? kk : 0, xv, xg);
            if constexpr (QW && WT::kBits == 4) {
                // The lane's 32 values are one block: acc += d * (sum(q x) - 8 sum(x)) (Q4_0) or
                // d * sum(q x) + m * sum(x) (Q4_1), with d = m = 0 past K and sum(x) the block sum
                // staged beside the activations. Each nibble is masked in place into an fp16 lane
                // of a pair, where it reads as the subnormal q * 2^-24 (bits 0-3) or q * 2^-20
                // (bits 4-7), and v_fma_mix multiplies it by the fp32 activation exactly as a
                // converted integer would be: products of the two bit positions go to separate
                // sums, rescaled by 2^24 and 2^20 once per block.
                const float xsum = xs[a.K + (in ? kk : 0) / 32];
#pragma unroll
                for (int r = 0; r < R; ++r) {
                    const uint32_t wd[4] = {w[r][u].x, w[r][u].y, w[r][u].z, w[r][u].w};
                    float s0 = 0.f, s1 = 0.f;
#pragma unroll
                    for (int m = 0; m < 4; ++m) {
                        // dword m holds values 8m .. 8m+7: value 2b in the low, 2b+1 in the high
                        // nibble of byte b; the pairs are (8m, 8m+4), (8m+1, 8m+5) from the
                        // dword, (8m+2, 8m+6), (8m+3, 8m+7) from the dword shifted by one byte
                        const uint32_t t = wd[m] >> 8;
                        const half2v p0 = __builtin_bit_cast(half2v, wd[m] & 0x000F000Fu);
                        const half2v p1 = __builtin_bit_cast(half2v, wd[m] & 0x00F000F0u);
                        const half2v p2 = __builtin_bit_cast(half2v, t & 0x000F000Fu);
                        const half2v p3 = __builtin_bit_cast(half2v, t & 0x00F000F0u);
                        const float* xm = xv + 8 * m;
                        s0 = fmaf((float)p0[0], xm[0], s0);
                        s0 = fmaf((float)p0[1], xm[4], s0);
                        s0 = fmaf((float)p2[0], xm[2], s0);
                        s0 = fmaf((float)p2[1], xm[6], s0);
                        s1 = fmaf((float)p1[0], xm[1], s1);
                        s1 = fmaf((float)p1[1], xm[5], s1);
                        s1 = fmaf((float)p3[0], xm[3], s1);
                        s1 = fmaf((float)p3[1], xm[7], s1);
                    }
                    const float b = fmaf(s1, 0x1p20f, s0 * 0x1p24f);  // sum(q x)
                    const float d = in ? qs[r][u] : 0.f;
                    if constexpr (WT::kMin) {
                        acc[r] = fmaf(d, b, acc[r]);
                        acc[r] = fmaf(in ? qm[r][u] : 0.f, xsum, acc[r]);
                    } else {
                        acc[r] = fmaf(d, fmaf(-8.f, xsum, b), acc[r]);
                    }
                }
                continue;
            }
            if constexpr (QW) {
                // Q8: two lanes share a block; acc += d * sum(q x), with d = 0 past K
#pragma unroll
                for (int r = 0; r < R; ++r) {
                    float wf[VEC];
                    unpack(w[r][u], WT(), wf);
                    float b = 0.f;
#pragma unroll
                    for (int i = 0; i < VEC; ++i) b = fmaf(wf[i], xv[i], b);
                    acc[r] = fmaf(in ? qs[r][u] : 0.f, b, acc[r]);
                }
                continue;
            }
#pragma unroll
            for (int r = 0; r < R; ++r) {
                const uint4 wr = in ? w[r][u] : make_uint4(0u, 0u, 0u, 0u);
                float wf[VEC];
                unpack(wr, WT(), wf);
#pragma unroll
                for (int i = 0; i < VEC; ++i) acc[r] = fmaf(wf[i], xv[i], acc[r]);
            }
        }
        if constexpr (EPI == EPI_RESID || EPI == EPI_QKV) {
#pragma unroll
            for (int r = 0; r < R; ++r) asm volatile("" ::"v"(pf[r]));
        }
        if (c == cpg - 1) epilogue(g0 + gi * stride, pf);
    };

    // Prologue: activation and gain loads, then the first weight tile, then the control block; the
    // staging, the norm and the control-block latency all complete under the weight fetch.
    XStage<WAVES, XPT> st;
    st.load(a.x, a.xh, a.gamma, a.K);
    uint4 wa[R][U], wb[R][U];
    float sa[R][U], sb[R][U], ma[R][U], mb[R][U];  // block scales / offsets of a quantized pack
    float pa[R], pb[R];
    issue_w(wa, sa, ma, 0);
    issue_w(wb, sb, mb, 1);
    __builtin_amdgcn_sched_barrier(0);
    if (a.ctrl) {
        if (a.ctrl->done) return;
        pos = a.ctrl->pos;
    }
    if constexpr (EPI == EPI_QKV) {
        if (pos >= a.cap) {
            if (blockIdx.x == 0 && threadIdx.x == 0) {
                a.ctrl->error = 1u;
                a.ctrl->done = 1u;
            }
            return;
        }
    }
    issue_pf(pa, 0);  // the RoPE angles depend on pos
    issue_pf(pb, 1);
    st.template store<xs_swizzled<WT>(), QW && WT::kBits == 4>(a.gamma, a.eps, a.K, xs, red);

    // Straight-line pairs with a single loop exit: the compiler's memory-counter waits merge over
    // every control-flow edge, so a conditional issue, a skipped consume or a mid-loop exit would
    // leave a buffer's loads pending on some edge and serialise the pipeline. Both buffers are
    // requested before the staging, so two tiles are in flight from the start; a buffer is refilled
    // right after it is consumed, and the last pair (peeled) is consumed without refills, so no
    // load is outstanding when the wave ends. An odd tile count is padded with one tile past the
    // wave's last group, and a wave without groups consumes one pair of such tiles (clamped
    // addresses, no output rows).
    const uint32_t n_pairs = n_tiles ? (n_tiles + 1) / 2 : 1;
    // (sched_barrier: keep each issue ahead of the next tile's arithmetic in the schedule)
    for (uint32_t p = 0; p + 1 < n_pairs; ++p) {
        consume(wa, sa, ma, pa, 2 * p);
        issue(wa, sa, ma, pa, 2 * p + 2);
        __builtin_amdgcn_sched_barrier(0);
        consume(wb, sb, mb, pb, 2 * p + 1);
        issue(wb, sb, mb, pb, 2 * p + 3);
        __builtin_amdgcn_sched_barrier(0);
    }
    consume(wa, sa, ma, pa, 2 * n_pairs - 2);
    consume(wb, sb, mb, pb, 2 * n_pairs - 1);

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
            for (int w = 1; w < WAVES; ++w) argmax_merge(v, i, bval[w], bidx[w]);
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

// Upper bound on a decode GEMV's grid: blocks-per-CU x the current device's CU count, by default the
// blocks that keep 16 waves per CU (one resident round), 8 for the QKV GEMV (measured on the 8B
// step at 8 / 12 / 16 / 24 / 32 waves per CU and no bound: QKV 10.08 / 10.69 / 10.64 / 10.67 /
// 10.67 / 10.65 us, the other GEMVs best or level at 16); VSL_GEMV_BLOCKS_PER_CU overrides it for
// every GEMV and 0 removes the bound. A bounded grid strides over the row groups, staging the
// activation vector once per block instead of once per few groups.
uint32_t gemv_grid_cap(int waves, int epi) {
    static int per_cu_env = -2;
    if (per_cu_env == -2) {
        const char* e = getenv("VSL_GEMV_BLOCKS_PER_CU");
        per_cu_env = e ? atoi(e) : -1;
        if (e && per_cu_env < 0) per_cu_env = 0;
    }
    const int resident = epi == EPI_QKV ? 8 : 16;  // default waves per CU
    const int per_cu = per_cu_env >= 0 ? per_cu_env : (waves >= resident ? 1 : resident / waves);
    if (per_cu == 0) return 0xFFFFFFFFu;
    static int cus[64] = {0};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 0xFFFFFFFFu;
    if (cus[dev] == 0) {
        int n = 0;
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
        cus[dev] = n;
    }
    return (uint32_t)per_cu * (uint32_t)cus[dev];
}

template <int R, int EPI, int WAVES>
uint32_t gemv_blocks(uint32_t N, uint32_t max_blocks) {
    constexpr int RG = (EPI == EPI_SWIGLU) ? R / 2 : R;
    const uint32_t groups = (N + RG - 1) / RG;
    uint32_t blocks = (groups + WAVES - 1) / WAVES;
    if (blocks > max_blocks) blocks = max_blocks;
    const uint32_t cap = gemv_grid_cap(WAVES, EPI);
    if (blocks > cap) blocks = cap;
    return blocks == 0 ? 1 : blocks;
}

constexpr uint32_t kMaxK = 32768;  // activation vector held in LDS as fp32 (up to 128 KB)

// XPT: float4 of the activation vector staged per thread, the smallest power of two covering K
template <class WT, int R, int U, int EPI, int WAVES, class ET = WF32>
int launch_gemv(const GemvArgs& a, uint32_t max_blocks, hipStream_t s) {
    const uint32_t blocks = gemv_blocks<R, EPI, WAVES>(a.N, max_blocks);
    // the fp32 activation vector, and for 4-bit packs its 32-value block sums
    const size_t lds = (size_t)xs_floats(a.K) * sizeof(float) + (WT::kBits == 4 ? (size_t)a.K / 32 * sizeof(float) : 0);
    const uint32_t per = WAVES * 64 * 4;
    if (a.K <= per)
        k_gemv_dec<WT, R, U, EPI, ET, WAVES, 1><<<blocks, WAVES * 64, lds, s>>>(a);
    else if (a.K <= 2 * per)
        k_gemv_dec<WT, R, U, EPI, ET, WAVES, 2><<<blocks, WAVES * 64, lds, s>>>(a);
    else if (a.K <= 4 * per)
        k_gemv_dec<WT, R, U, EPI, ET, WAVES, 4><<<blocks, WAVES * 64, lds, s>>>(a);
    else if (WAVES * 64 * 4 * 4 < kMaxK && a.K <= 8 * per)
        k_gemv_dec<WT, R, U, EPI, ET, WAVES, (WAVES * 64 * 4 * 4 < kMaxK ? 8 : 4)><<<blocks, WAVES * 64, lds, s>>>(a);
    else
        return vsl_invalid("decode GEMV: K=%u exceeds the %u-wave staging", a.K, (unsigned)WAVES);
    HIP_TRY(hipGetLastError());
    return VSL_OK;
}

// Block size by K: the fp32 activation vector takes K*4 bytes of LDS per block; past 8192
// columns, 8-wave blocks keep 16 waves resident per CU within the 160 KB of LDS; past 16384 (the
// down projection of 70B-class FFNs, 28672), one 16-wave block per CU holds up to 128 KB.
constexpr uint32_t kWideK = 8192, kXWideK = 16384;

int gemv_waves_env() {
    static int w = -1;
    if (w < 0) {
        const char* e = getenv("VSL_GEMV_WAVES");
        w = e ? atoi(e) : 0;
        if (w != 4 && w != 8 && w != 16) w = 0;
    }
    return w;
}

template <class WT, int R, int U, int EPI, class ET = WF32>
int launch_gemv_k(const GemvArgs& a, uint32_t max_blocks, hipStream_t s) {
    switch (gemv_waves_env()) {
        case 16: return launch_gemv<WT, R, U, EPI, 16, ET>(a, max_blocks, s);
        case 8: if (a.K <= kXWideK) return launch_gemv<WT, R, U, EPI, 8, ET>(a, max_blocks, s); break;
        case 4: if (a.K <= kWideK) return launch_gemv<WT, R, U, EPI, 4, ET>(a, max_blocks, s); break;
        default: break;
    }
    if (a.K > kXWideK) return launch_gemv<WT, R, U, EPI, 16, ET>(a, max_blocks, s);
    return a.K > kWideK ? launch_gemv<WT, R, U, EPI, 8, ET>(a, max_blocks, s)
                        : launch_gemv<WT, R, U, EPI, 4, ET>(a, max_blocks, s);
}

template <int R, int EPI>
uint32_t gemv_blocks_k(uint32_t N, uint32_t K, uint32_t max_blocks) {
    // the grid launch_gemv_k chooses
    switch (gemv_waves_env()) {
        case 16: return gemv_blocks<R, EPI, 16>(N, max_blocks);
        case 8: if (K <= kXWideK) return gemv_blocks<R, EPI, 8>(N, max_blocks); break;
        case 4: if (K <= kWideK) return gemv_blocks<R, EPI, 4>(N, max_blocks); break;
        default: break;
    }
    if (K > kXWideK) return gemv_blocks<R, EPI, 16>(N, max_blocks);
    return K > kWideK ? gemv_blocks<R, EPI, 8>(N, max_blocks) : gemv_blocks<R, EPI, 4>(N, max_blocks);
}


int check_gemv_shape(uint32_t N, uint32_t K, const char* who) {
    if (N == 0 || K == 0) return vsl_invalid("%s: empty shape", who);
    if (K % 8) return vsl_invalid("%s: K=%u must be a multiple of 8", who, K);
    if (K > kMaxK) return vsl_invalid("%s: K=%u exceeds %u", who, K, kMaxK);
    return VSL_OK;
}

bool quant_dtype(int wdtype) { return wdtype == VSL_DT_Q8_0 || wdtype == VSL_DT_Q4_0 || wdtype == VSL_DT_Q4_1; }

// Block-quantized packs: every block stages the whole fp32 activation vector (4 bytes per column) for weights of
// 0.56 - 1.13 bytes per value, so that with the fp16 launch shapes the staging traffic approaches the
// weight bytes where a block covers few rows. Larger blocks (fewer of them, each CU's resident waves
// sharing one copy) measured faster for the SwiGLU GEMV (8 waves) and the residual GEMV from 8192
// input columns (16 waves); kernel-trace medians, Q4_0 / Q8_0, fp16 shape -> this one: 8B gate/up
// 15.9 -> 14.6 / 23.0 -> 22.3 us, 8B down 11.2 -> 10.4 / 13.5 -> 13.4 us, 70B-class O projection
// (8192 x 8192) 13.1 -> 11.6 us for Q4_0. The QKV GEMV (4 waves: 6.5 / 7.4 us against 7.1 / 8.5 at
// 8), the 8B O projection (K 4096: level within 0.3 us at 4, 8 or 16 waves for Q4_0; 5.6 at 4 against
// 6.3 at 16 for Q8_0) and lm_head keep the fp16 shapes. Two rows per wave in those residual GEMVs:
// 70B-class down projection (8192 rows) 30.5 -> 28.0 us, O 11.3 -> 11.1 us; with 4096 rows (8B: half
// the waves idle) 10.4 -> 13.4 / 13.6 -> 17.4 us, so only from 8192 rows.
template <class WT, int R, int U, int EPI, class ET>
int launch_gemv_q(const GemvArgs& a, uint32_t max_blocks, hipStream_t s) {
    if (gemv_waves_env() == 0) {
        if constexpr (EPI == EPI_SWIGLU) {
            if (a.K <= kXWideK) return launch_gemv<WT, R, U, EPI, 8, ET>(a, max_blocks, s);
        } else if constexpr (EPI == EPI_RESID) {
            if (a.K >= kWideK) {
                // two rows per wave once the rows fill every resident wave twice over (each staged
                // activation read then serves two rows)
                if constexpr (R == 1) {
                    if ((uint64_t)a.N >= 2ull * 16ull * gemv_grid_cap(16, EPI_RESID))
                        return launch_gemv<WT, 2, U, EPI, 16, ET>(a, max_blocks, s);
                }
                return launch_gemv<WT, R, U, EPI, 16, ET>(a, max_blocks, s);
            }
        }
    }
    return launch_gemv_k<WT, R, U, EPI, ET>(a, max_blocks, s);
}

// The decode GEMV over the weight dtype: fp16 / fp32 matrices with four 16-byte loads per lane and row
// per tile; block-quantized packs with the same 2048 columns per tile (Q8: two loads of 16 values,
// Q4: one of 32).
template <int R, int EPI, class ET = WF32>
int launch_gemv_w(int wdtype, const GemvArgs& a, uint32_t max_blocks, hipStream_t s, const char* who) {
    if (quant_dtype(wdtype)) {
        if (a.K % 32) return vsl_invalid("%s: a block-quantized pack needs K %% 32 == 0 (K=%u)", who, a.K);
        if (reinterpret_cast<uintptr_t>(a.W) & 255) return vsl_invalid("%s: a block-quantized pack must be 256-byte aligned", who);
    }
    switch (wdtype) {
        case VSL_DT_F16: return launch_gemv_k<WF16, R, 4, EPI, ET>(a, max_blocks, s);
        case VSL_DT_F32: return launch_gemv_k<WF32, R, 4, EPI, ET>(a, max_blocks, s);
        case VSL_DT_Q8_0: return launch_gemv_q<WQ8, R, 2, EPI, ET>(a, max_blocks, s);
        case VSL_DT_Q4_0: return launch_gemv_q<WQ4, R, 1, EPI, ET>(a, max_blocks, s);
        case VSL_DT_Q4_1: return launch_gemv_q<WQ41, R, 1, EPI, ET>(a, max_blocks, s);
        default: return vsl_unsupported("%s: weight dtype %d", who, wdtype);
    }
}

// ---------------------------------------------------------------------------------------------
// flash-decode attention (split-KV, online softmax) + split combine
// ---------------------------------------------------------------------------------------------
constexpr float kLog2e = 1.4426950408889634f;

// Block (split s, KV head h), WAVES waves. A lane group of LPP lanes holds one position (8 head
// dims per lane), a wave SLOTS positions, the block NSLOT; a tile is P such rows of the block
// (P positions per lane, TILE positions), so P x 32 bytes per lane are in flight per tile. Block s
// owns tiles s, s + nsplit, s + 2 nsplit, ... A block's tile addresses do not depend on the
// sequence length, so its first two tiles are requested before the control block is read, and
// every next tile before the current one is consumed (two register buffers, as in the GEMV).
// Positions at or past the length are masked by selects; their loads read position 0.
//
// WIN: the windowed mode. The query at position p attends to every key k <= p while p + 1 <= thr;
// past that, to the n_glob first keys and the win keys before p (k >= p - win) only. The tiles
// then run over that set as virtual positions v (v < n_glob -> k = v, else k = v + p - win - n_glob),
// which depend on p, so the first tiles are requested after the control block is read.
//
// Output: the split's softmax partials per query head, part_ml = (m, l) and part_o = sum_k 2^(s_k - m)
// v_k (scores in log2 units), merged by k_attn_combine.
template <class KT, int HD, int G, bool WIN, int WAVES, int P>
__global__ __launch_bounds__(WAVES * 64) void k_attn_decode(const float* __restrict__ q, const void* __restrict__ kcache,
                                                            const void* __restrict__ vcache, uint32_t n_q, uint32_t n_kv,
                                                            uint32_t cap, float scale, uint32_t nsplit,
                                                            float* __restrict__ part_o, float* __restrict__ part_ml,
                                                            vsl_ctrl* ctrl, uint32_t win, uint32_t n_glob, uint32_t thr) {
    typedef typename KT::T T;
    constexpr int NT = WAVES * 64;
    constexpr int LPP = HD / 8;            // lanes per position, 8 elements per lane
    constexpr int SLOTS = 64 / LPP;        // positions per wave per row
    constexpr int NSLOT = WAVES * SLOTS;   // positions per row of the block
    constexpr uint32_t TILE = NSLOT * P;   // positions per tile
    constexpr int KW = sizeof(T) * 8 / 16; // 16-byte loads per lane per position (1 fp16, 2 fp32)
    __shared__ float s_ml[WAVES][G][2];
    __shared__ float s_acc[WAVES][G][HD];

    const uint32_t kvh = blockIdx.y, split = blockIdx.x;
    const uint32_t lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t slot = lane / LPP, sub = lane % LPP;
    const uint32_t h0 = kvh * G;  // first query head of this KV head (kv_head = head*n_kv/n_q)
    const T* Kb = static_cast<const T*>(kcache) + (size_t)kvh * cap * HD;
    const T* Vb = static_cast<const T*>(vcache) + (size_t)kvh * cap * HD;

    struct Tile {
        uint4 k[P][KW], v[P][KW];
    };
    uint32_t shift = 0;  // WIN: key position = virtual position + shift past the n_glob first keys
    auto position = [&](uint32_t j, int p) {
        return (j * nsplit + split) * TILE + (uint32_t)p * NSLOT + wave * SLOTS + slot;
    };
    // positions at or past `limit` read position 0 instead (in bounds, and the same cache lines
    // for every such lane)
    auto issue = [&](Tile& b, uint32_t j, uint32_t limit) {
#pragma unroll
        for (int p = 0; p < P; ++p) {
            uint32_t t = position(j, p);
            t = t < limit ? t : 0;
            if constexpr (WIN) t = t < n_glob ? t : t + shift;
            const T* kp = Kb + (size_t)t * HD + sub * 8;
            const T* vp = Vb + (size_t)t * HD + sub * 8;
#pragma unroll
            for (int w = 0; w < KW; ++w) {
                b.k[p][w] = load16<false>(kp + w * (8 / KW));
                b.v[p][w] = load16<false>(vp + w * (8 / KW));
            }
        }
    };

    // q and the first two tiles are requested before the control block is read. Both tiles are
    // consumed on every path and no branch depends on `done` (it only gates the stores), so the
    // compiler has no path to sink these loads into behind the control-block wait.
    float4 qr[G][2];
#pragma unroll
    for (int g = 0; g < G; ++g) {
        const float* qp = q + (size_t)(h0 + g) * HD + sub * 8;
        qr[g][0] = *reinterpret_cast<const float4*>(qp);
        qr[g][1] = *reinterpret_cast<const float4*>(qp + 4);
    }
    Tile ta, tb;
    if constexpr (!WIN) {
        issue(ta, 0, cap);
        issue(tb, 1, cap);
    }
    __builtin_amdgcn_sched_barrier(0);
    const uint32_t done = ctrl->done;
    const uint32_t pos = ctrl->pos;
    const uint32_t len = pos < cap ? pos + 1 : cap;  // pos >= cap only with done set
    // keys attended (virtual positions 0 .. n_att-1)
    uint32_t n_att = len;
    if constexpr (WIN) {
        const uint32_t p = len - 1;  // the query position (clamped with `len` when done)
        if (len > thr && p > n_glob + win) {  // otherwise the two ranges cover 0..p
            n_att = n_glob + win + 1;
            shift = p - win - n_glob;
        }
        issue(ta, 0, n_att);
        issue(tb, 1, n_att);
    }

    float qv[G][8];
#pragma unroll
    for (int g = 0; g < G; ++g) {
        const float4 a = qr[g][0], b = qr[g][1];
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

    // Per tile: the P scores of every head (DPP sums over the position's lane group), one running
    // maximum update and one rescale of the accumulators, then the P weighted values.
    auto consume = [&](const Tile& b, uint32_t j) {
        float kf[P][8], vf[P][8];
        bool valid[P];
#pragma unroll
        for (int p = 0; p < P; ++p) {
            valid[p] = position(j, p) < n_att;
            if constexpr (KW == 1) {
                unpack(b.k[p][0], KT(), kf[p]);
                unpack(b.v[p][0], KT(), vf[p]);
            } else {
                unpack(b.k[p][0], KT(), kf[p]);
                unpack(b.k[p][1], KT(), kf[p] + 4);
                unpack(b.v[p][0], KT(), vf[p]);
                unpack(b.v[p][1], KT(), vf[p] + 4);
            }
#pragma unroll
            for (int i = 0; i < 8; ++i) vf[p][i] = valid[p] ? vf[p][i] : 0.f;  // cache memory past len is arbitrary
        }
#pragma unroll
        for (int g = 0; g < G; ++g) {
            float sc[P];
            float mt = m[g];
#pragma unroll
            for (int p = 0; p < P; ++p) {
                float d = 0.f;
#pragma unroll
                for (int i = 0; i < 8; ++i) d = fmaf(qv[g][i], kf[p][i], d);
                sc[p] = group_sum_dpp<LPP>(d);
                mt = valid[p] ? fmaxf(mt, sc[p]) : mt;
            }
            // m = -inf: 0 (nothing accumulated yet); no valid key so far: keep (mt - mt would be NaN)
            const float corr = mt == -INFINITY ? 1.f : fast_exp2(m[g] - mt);
            float ls = 0.f;
#pragma unroll
            for (int i = 0; i < 8; ++i) acc[g][i] *= corr;
#pragma unroll
            for (int p = 0; p < P; ++p) {
                const float pr = valid[p] ? fast_exp2(sc[p] - mt) : 0.f;
                ls += pr;
#pragma unroll
                for (int i = 0; i < 8; ++i) acc[g][i] = fmaf(pr, vf[p][i], acc[g][i]);
            }
            l[g] = fmaf(l[g], corr, ls);
            m[g] = mt;
        }
    };

    const uint32_t total = (n_att + TILE - 1) / TILE;  // tiles holding positions < n_att
    const uint32_t mine = total > split ? (total - 1 - split) / nsplit + 1 : 0;
    // pairs with a single loop exit, each buffer refilled right after it is consumed; the last pair
    // (peeled) is consumed without refills so that no load is outstanding past it (tiles past the
    // block's own are masked: their positions are >= n_att)
    const uint32_t n_pairs = mine ? (mine + 1) / 2 : 1;
    for (uint32_t pp = 0; pp + 1 < n_pairs; ++pp) {
        consume(ta, 2 * pp);
        issue(ta, 2 * pp + 2, n_att);
        __builtin_amdgcn_sched_barrier(0);
        consume(tb, 2 * pp + 1);
        issue(tb, 2 * pp + 3, n_att);
        __builtin_amdgcn_sched_barrier(0);
    }
    consume(ta, 2 * n_pairs - 2);
    consume(tb, 2 * n_pairs - 1);

    // merge the wave's SLOTS position groups (lanes sub + LPP * slot hold the same dims): pairs of
    // lanes at distances LPP .. 32, merged symmetrically so that both lanes of a pair agree
    auto merge_pairs = [&](auto xc) {
        constexpr int X = decltype(xc)::value;
#pragma unroll
        for (int g = 0; g < G; ++g) {
            float ma, mb, la, lb;
            lane_pair<X>(m[g], ma, mb);
            lane_pair<X>(l[g], la, lb);
            const float M = fmaxf(ma, mb);
            const float fa = ma == -INFINITY ? 0.f : fast_exp2(ma - M);
            const float fb = mb == -INFINITY ? 0.f : fast_exp2(mb - M);
            l[g] = la * fa + lb * fb;
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                float aa, ab;
                lane_pair<X>(acc[g][i], aa, ab);
                acc[g][i] = aa * fa + ab * fb;
            }
            m[g] = M;
        }
    };
    if constexpr (LPP == 8) merge_pairs(std::integral_constant<int, 8>());
    merge_pairs(std::integral_constant<int, 16>());
    merge_pairs(std::integral_constant<int, 32>());
    if (slot == 0) {
#pragma unroll
        for (int g = 0; g < G; ++g) {
            if (sub == 0) {
                s_ml[wave][g][0] = m[g];
                s_ml[wave][g][1] = l[g];
            }
#pragma unroll
            for (int i = 0; i < 8; ++i) s_acc[wave][g][sub * 8 + i] = acc[g][i];
        }
    }
    lds_barrier();
    for (uint32_t e = threadIdx.x; e < (uint32_t)(G * HD); e += NT) {
        const uint32_t g = e / HD, dd = e % HD;
        float M = -INFINITY;
#pragma unroll
        for (int w = 0; w < WAVES; ++w) M = fmaxf(M, s_ml[w][g][0]);
        float L = 0.f, A = 0.f;
        if (M != -INFINITY) {
#pragma unroll
            for (int w = 0; w < WAVES; ++w) {
                const float f = exp2f(s_ml[w][g][0] - M);
                L += s_ml[w][g][1] * f;
                A += s_acc[w][g][dd] * f;
            }
        }
        const size_t pidx = (size_t)(h0 + g) * nsplit + split;
        if (!done) {
            part_o[pidx * HD + dd] = A;
            if (dd == 0) {
                part_ml[pidx * 2 + 0] = M;
                part_ml[pidx * 2 + 1] = L;
            }
        }
    }
}

// Flash-decode on the matrix cores, for fp16 caches with head_dim 128 and G <= 8 query heads per KV
// head. Block (split s, KV head h) of WAVES waves; a wave owns 16-position tiles: block tile j holds
// positions [(j * nsplit + s) * 16 WAVES, + 16 WAVES), wave w the w-th 16 of them. Per tile:
//  - scores S = Q K^T by v_mfma_f32_16x16x32_f16 over the four 32-dim k-steps, twice: A = the G query
//    rows (zero-padded to 16) as the hi and the lo fp16 planes of q * scale * log2(e), so the products
//    are those of the fp32 q; B = the tile's K rows, lane l holding position l % 16, dims
//    32 ks + 8 (l / 16) .. + 7 (its own 16-byte loads). D holds head 4 (l / 16) + i, position l % 16
//    in register i of lane l, so each head's 16 scores lie on one 16-lane row;
//  - the online softmax of each head on its row (DPP maximum, exp2): the running maximum is the same
//    in every lane of the row, the running sum is kept per lane and summed over the row at the end;
//  - the probabilities and each head's rescale factor go through the wave's 1 KB of LDS to every
//    lane, and lane l accumulates head dims 2l and 2l + 1 of every head from its 4-byte V loads (a
//    256-byte cache row per load instruction), fp32 FMAs on the fp16 values.
// Against k_attn_decode (16 lanes per position, 8 dims per lane) a wave handles 16 positions per tile
// instead of 4 and drops the per-head lane-group sums. Tiles are requested two ahead in registers as
// there; positions at or past the length load position 0 and get probability 0. The output is
// k_attn_decode's: per head of the split, (m, l) and the unnormalised sum, merged by k_attn_combine.
template <int G, int WAVES>
__global__ __launch_bounds__(WAVES * 64) void k_attn_decode_mfma(const float* __restrict__ q,
                                                                 const vsl_half* __restrict__ kcache,
                                                                 const vsl_half* __restrict__ vcache, uint32_t cap,
                                                                 float scale, uint32_t nsplit,
                                                                 float* __restrict__ part_o,
                                                                 float* __restrict__ part_ml, vsl_ctrl* ctrl) {
    constexpr int HD = 128, KS = HD / 32, TP = 16;  // k-steps, positions per wave tile
    constexpr uint32_t TB = TP * WAVES;             // positions per block tile
    constexpr int NR = (G + 3) / 4;                 // 16-lane rows holding heads (four per row)
    static_assert(G >= 1 && G <= 8, "GQA group of 1..8 heads");
    __shared__ __attribute__((aligned(16))) float s_p[WAVES][TP][8];  // probabilities [position][head]
    __shared__ __attribute__((aligned(16))) float s_c[WAVES][8];      // rescale factor per head
    __shared__ float s_ml[WAVES][G][2];
    __shared__ float s_acc[WAVES][G][HD];

    const uint32_t kvh = blockIdx.y, split = blockIdx.x;
    const uint32_t lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t col = lane & 15, rg = lane >> 4;  // MFMA column (tile position / A row), row group
    const uint32_t h0 = kvh * G;
    const vsl_half* Kb = kcache + (size_t)kvh * cap * HD;
    const vsl_half* Vb = vcache + (size_t)kvh * cap * HD;

    struct Tile {
        uint4 k[KS];
        uint32_t v[TP];
    };
    auto tile_pos = [&](uint32_t j) { return (j * nsplit + split) * TB + wave * TP; };
    // positions at or past `limit` read position 0 instead (in bounds)
    auto issue = [&](Tile& b, uint32_t j, uint32_t limit) {
        const uint32_t p0 = tile_pos(j);
        const uint32_t t = p0 + col < limit ? p0 + col : 0;
        const vsl_half* kp = Kb + (size_t)t * HD + rg * 8;
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) b.k[ks] = load16<false>(kp + 32 * ks);
#pragma unroll
        for (int i = 0; i < TP; ++i) {
            const uint32_t tv = p0 + i < limit ? p0 + i : 0;
            b.v[i] = *reinterpret_cast<const uint32_t*>(Vb + (size_t)tv * HD + 2 * lane);
        }
    };

    // A operands (lane l: query row l % 16, dims 32 ks + 8 (l / 16) .. + 7), requested with the first
    // two tiles before the control block is read
    float4 qa[KS][2];
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
        if (col < (uint32_t)G) {
            const float* qp = q + (size_t)(h0 + col) * HD + 32 * ks + 8 * rg;
            qa[ks][0] = *reinterpret_cast<const float4*>(qp);
            qa[ks][1] = *reinterpret_cast<const float4*>(qp + 4);
        } else {
            qa[ks][0] = qa[ks][1] = make_float4(0.f, 0.f, 0.f, 0.f);
        }
    }
    Tile ta, tb;
    issue(ta, 0, cap);
    issue(tb, 1, cap);
    __builtin_amdgcn_sched_barrier(0);
    const uint32_t done = ctrl->done;
    const uint32_t pos = ctrl->pos;
    const uint32_t n_att = pos < cap ? pos + 1 : cap;  // pos >= cap only with done set

    half8 qh[KS], ql[KS];
    const float f = scale * kLog2e;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
        const float x[8] = {qa[ks][0].x * f, qa[ks][0].y * f, qa[ks][0].z * f, qa[ks][0].w * f,
                            qa[ks][1].x * f, qa[ks][1].y * f, qa[ks][1].z * f, qa[ks][1].w * f};
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            vsl_half hi, lo;
            split_f16(x[e], hi, lo);
            qh[ks][e] = hi;
            ql[ks][e] = lo;
        }
    }
    float m[4], ls[4], acc[G][2];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        m[i] = -INFINITY;
        ls[i] = 0.f;
    }
#pragma unroll
    for (int g = 0; g < G; ++g) acc[g][0] = acc[g][1] = 0.f;

    auto consume = [&](const Tile& b, uint32_t j) {
        float4v s = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
            const half8 kk = __builtin_bit_cast(half8, b.k[ks]);
            s = __builtin_amdgcn_mfma_f32_16x16x32_f16(qh[ks], kk, s, 0, 0, 0);
            s = __builtin_amdgcn_mfma_f32_16x16x32_f16(ql[ks], kk, s, 0, 0, 0);
        }
        const bool valid = tile_pos(j) + col < n_att;
        float pr[4], corr[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float x = valid ? s[i] : -INFINITY;
            const float mn = fmaxf(m[i], row_max16_dpp(x));
            // mn = -inf: no valid key in this row yet (everything is still 0)
            corr[i] = mn == -INFINITY ? 1.f : fast_exp2(m[i] - mn);
            pr[i] = valid ? fast_exp2(x - mn) : 0.f;
            ls[i] = fmaf(ls[i], corr[i], pr[i]);
            m[i] = mn;
        }
        if (rg < (uint32_t)NR) {
            *reinterpret_cast<float4*>(&s_p[wave][col][4 * rg]) = make_float4(pr[0], pr[1], pr[2], pr[3]);
            if (col == 0) *reinterpret_cast<float4*>(&s_c[wave][4 * rg]) = make_float4(corr[0], corr[1], corr[2], corr[3]);
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront", "local");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront", "local");
        float c[8];
        *reinterpret_cast<float4*>(c) = *reinterpret_cast<const float4*>(&s_c[wave][0]);
        if constexpr (G > 4) *reinterpret_cast<float4*>(c + 4) = *reinterpret_cast<const float4*>(&s_c[wave][4]);
#pragma unroll
        for (int g = 0; g < G; ++g) {
            acc[g][0] *= c[g];
            acc[g][1] *= c[g];
        }
        const uint32_t p0 = tile_pos(j);
#pragma unroll
        for (int i = 0; i < TP; ++i) {
            float pp[8];
            *reinterpret_cast<float4*>(pp) = *reinterpret_cast<const float4*>(&s_p[wave][i][0]);
            if constexpr (G > 4) *reinterpret_cast<float4*>(pp + 4) = *reinterpret_cast<const float4*>(&s_p[wave][i][4]);
            // the first two tiles were requested up to the capacity: cache rows past the length hold
            // arbitrary bits (possibly Inf / NaN), and 0 * NaN would reach the sum
            const uint32_t vbits = p0 + i < n_att ? b.v[i] : 0u;
            const half2v vv = __builtin_bit_cast(half2v, vbits);
            const float v0 = (float)vv[0], v1 = (float)vv[1];
#pragma unroll
            for (int g = 0; g < G; ++g) {
                acc[g][0] = fmaf(pp[g], v0, acc[g][0]);
                acc[g][1] = fmaf(pp[g], v1, acc[g][1]);
            }
        }
        // every lane has read this tile's values before the next tile's stores
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront", "local");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront", "local");
    };

    const uint32_t total = (n_att + TB - 1) / TB;  // block tiles holding positions < n_att
    const uint32_t mine = total > split ? (total - 1 - split) / nsplit + 1 : 0;
    // pairs with a single loop exit; the last pair (peeled) is consumed without refills so that no
    // load is outstanding past it (tiles past the block's own are masked: positions >= n_att)
    const uint32_t n_pairs = mine ? (mine + 1) / 2 : 1;
    for (uint32_t pp = 0; pp + 1 < n_pairs; ++pp) {
        consume(ta, 2 * pp);
        issue(ta, 2 * pp + 2, n_att);
        __builtin_amdgcn_sched_barrier(0);
        consume(tb, 2 * pp + 1);
        issue(tb, 2 * pp + 3, n_att);
        __builtin_amdgcn_sched_barrier(0);
    }
    consume(ta, 2 * n_pairs - 2);
    consume(tb, 2 * n_pairs - 1);

    // the wave's totals: sums over each row, maxima already row-uniform
#pragma unroll
    for (int i = 0; i < 4; ++i) ls[i] = group_sum_dpp<16>(ls[i]);
    if (col == 0 && rg < (uint32_t)NR) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t g = 4 * rg + i;
            if (g < (uint32_t)G) {
                s_ml[wave][g][0] = m[i];
                s_ml[wave][g][1] = ls[i];
            }
        }
    }
#pragma unroll
    for (int g = 0; g < G; ++g) *reinterpret_cast<float2*>(&s_acc[wave][g][2 * lane]) = make_float2(acc[g][0], acc[g][1]);
    lds_barrier();
    for (uint32_t e = threadIdx.x; e < (uint32_t)(G * HD); e += WAVES * 64) {
        const uint32_t g = e / HD, dd = e % HD;
        float M = -INFINITY;
#pragma unroll
        for (int w = 0; w < WAVES; ++w) M = fmaxf(M, s_ml[w][g][0]);
        float L = 0.f, A = 0.f;
        if (M != -INFINITY) {
#pragma unroll
            for (int w = 0; w < WAVES; ++w) {
                const float fw = exp2f(s_ml[w][g][0] - M);
                L += s_ml[w][g][1] * fw;
                A += s_acc[w][g][dd] * fw;
            }
        }
        const size_t pidx = (size_t)(h0 + g) * nsplit + split;
        if (!done) {
            part_o[pidx * HD + dd] = A;
            if (dd == 0) {
                part_ml[pidx * 2 + 0] = M;
                part_ml[pidx * 2 + 1] = L;
            }
        }
    }
}

// Combines the nsplit partials of every query head: out = sum_s A_s 2^(m_s-M) / sum_s l_s 2^(m_s-M).
// One block per head, one thread per head dim. With NS > 0 (nsplit <= NS <= 64) every partial is
// requested at once (before the control block is read) and held in registers, and wave 0 alone
// forms the split weights -- one split per lane, maximum and sum by DPP -- behind a single barrier;
// NS = 0 loops over any split count.
constexpr int kCombineThreads = 128;
constexpr uint32_t kMaxSplits = 1024;
constexpr int kFastSplits = 64;
template <int HD, int NS>
__global__ __launch_bounds__(kCombineThreads) void k_attn_combine(const float* __restrict__ part_o,
                                                                  const float* __restrict__ part_ml, uint32_t nsplit,
                                                                  float* __restrict__ out, const vsl_ctrl* ctrl) {
    static_assert(NS == 0 || (NS % 4 == 0 && NS <= 64), "register path: up to 64 splits in wave 0");
    __shared__ float wts[NS > 0 ? NS : kMaxSplits];
    __shared__ float red[kCombineThreads / 64];
    __shared__ float s_M, s_L;
    const uint32_t h = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const size_t base = (size_t)h * nsplit;
    const uint32_t dd = tid < (uint32_t)HD ? tid : 0;
    float a0 = 0.f, a1 = 0.f, a2 = 0.f, a3 = 0.f;
    uint32_t done;
    if constexpr (NS > 0) {
        float m0 = -INFINITY, l0 = 0.f;
        if (tid < nsplit) {
            m0 = part_ml[(base + tid) * 2];
            l0 = part_ml[(base + tid) * 2 + 1];
        }
        float o[NS];
#pragma unroll
        for (int s = 0; s < NS; ++s) o[s] = part_o[(base + (s < (int)nsplit ? s : 0)) * HD + dd];
        done = ctrl->done;  // gates the store only (no branch to sink the loads behind)
        if (wave == 0) {    // lanes past nsplit hold m = -inf and weight 0
            const float M = wave_max_dpp(m0);
            const float f = m0 == -INFINITY ? 0.f : exp2f(m0 - M);
            if (tid < (uint32_t)NS) wts[tid] = f;
            const float L = wave_sum_dpp(l0 * f);
            if (lane == 0) s_L = L;
        }
        __syncthreads();
#pragma unroll
        for (int s = 0; s < NS; s += 4) {
            a0 = fmaf(o[s], wts[s], a0);
            a1 = fmaf(o[s + 1], wts[s + 1], a1);
            a2 = fmaf(o[s + 2], wts[s + 2], a2);
            a3 = fmaf(o[s + 3], wts[s + 3], a3);
        }
    } else {
        done = ctrl->done;
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
        if (tid < (uint32_t)HD) {
            uint32_t s = 0;
            for (; s + 4 <= nsplit; s += 4) {
                a0 = fmaf(part_o[(base + s) * HD + dd], wts[s], a0);
                a1 = fmaf(part_o[(base + s + 1) * HD + dd], wts[s + 1], a1);
                a2 = fmaf(part_o[(base + s + 2) * HD + dd], wts[s + 2], a2);
                a3 = fmaf(part_o[(base + s + 3) * HD + dd], wts[s + 3], a3);
            }
            for (; s < nsplit; ++s) a0 = fmaf(part_o[(base + s) * HD + dd], wts[s], a0);
        }
    }
    if (tid >= (uint32_t)HD) return;
    const float inv = 1.0f / s_L;
    if (!done) out[(size_t)h * HD + dd] = ((a0 + a1) + (a2 + a3)) * inv;
}

struct AttnWindow {
    bool on;
    uint32_t win, n_glob, thr;
};

// Launch shape of k_attn_decode: 4 waves, one position per lane per tile (measured on the 8B
// workload against 4 x 2, 8 x 1 and 8 x 2 at 1K and 8K context: more positions per block lengthen
// the per-block latency chain more than they save in block count).
constexpr int kAttnWaves = 4, kAttnP = 1;
// Caches of more than kAttnMfmaMinCap positions (fp16, head_dim 128, dense) take k_attn_decode_mfma
// with 4 waves per block. Attention kernel alone at 32 splits, 8B shapes: 600 / 2000 / 8200 / 16000 /
// 32000 positions 5.25 / 6.11 / 11.60 / 16.63 / 28.86 us for k_attn_decode and 6.05 / 6.09 / 9.51 /
// 14.05 / 22.42 us for k_attn_decode_mfma: the launch is captured before the length is known, so
// the capacity picks the kernel.
constexpr uint32_t kAttnMfmaMinCap = 8192;
constexpr int kAttnMfmaWaves = 4;

template <class KT, int HD, int G, bool WIN, int WAVES, int P>
void launch_attn_shape(dim3 grid, hipStream_t s, const float* q, const void* kc, const void* vc, uint32_t n_q,
                       uint32_t n_kv, uint32_t cap, float scale, uint32_t nsplit, float* po, float* pml,
                       vsl_ctrl* ctrl, const AttnWindow& w) {
    k_attn_decode<KT, HD, G, WIN, WAVES, P><<<grid, WAVES * 64, 0, s>>>(q, kc, vc, n_q, n_kv, cap, scale, nsplit, po,
                                                                        pml, ctrl, w.win, w.n_glob, w.thr);
}

template <class KT, int HD, int G>
void launch_attn_w(dim3 grid, hipStream_t s, const float* q, const void* kc, const void* vc, uint32_t n_q,
                   uint32_t n_kv, uint32_t cap, float scale, uint32_t nsplit, float* po, float* pml, vsl_ctrl* ctrl,
                   const AttnWindow& w) {
    if constexpr (HD == 128 && G <= 8 && sizeof(typename KT::T) == 2) {
        if (!w.on && cap > kAttnMfmaMinCap) {
            k_attn_decode_mfma<G, kAttnMfmaWaves><<<grid, kAttnMfmaWaves * 64, 0, s>>>(
                q, static_cast<const vsl_half*>(kc), static_cast<const vsl_half*>(vc), cap, scale, nsplit, po, pml, ctrl);
            return;
        }
    }
    if (w.on)
        launch_attn_shape<KT, HD, G, true, kAttnWaves, kAttnP>(grid, s, q, kc, vc, n_q, n_kv, cap, scale, nsplit, po, pml,
                                                               ctrl, w);
    else
        launch_attn_shape<KT, HD, G, false, kAttnWaves, kAttnP>(grid, s, q, kc, vc, n_q, n_kv, cap, scale, nsplit, po,
                                                                pml, ctrl, w);
}

template <class KT, int HD>
int launch_attn_g(uint32_t G, dim3 grid, hipStream_t s, const float* q, const void* kc, const void* vc, uint32_t n_q,
                  uint32_t n_kv, uint32_t cap, float scale, uint32_t nsplit, float* po, float* pml, float* out,
                  vsl_ctrl* ctrl, const AttnWindow& w) {
    switch (G) {
        case 1: launch_attn_w<KT, HD, 1>(grid, s, q, kc, vc, n_q, n_kv, cap, scale, nsplit, po, pml, ctrl, w); break;
        case 2: launch_attn_w<KT, HD, 2>(grid, s, q, kc, vc, n_q, n_kv, cap, scale, nsplit, po, pml, ctrl, w); break;
        case 4: launch_attn_w<KT, HD, 4>(grid, s, q, kc, vc, n_q, n_kv, cap, scale, nsplit, po, pml, ctrl, w); break;
        case 3: launch_attn_w<KT, HD, 3>(grid, s, q, kc, vc, n_q, n_kv, cap, scale, nsplit, po, pml, ctrl, w); break;
        case 5: launch_attn_w<KT, HD, 5>(grid, s, q, kc, vc, n_q, n_kv, cap, scale, nsplit, po, pml, ctrl, w); break;
        case 6: launch_attn_w<KT, HD, 6>(grid, s, q, kc, vc, n_q, n_kv, cap, scale, nsplit, po, pml, ctrl, w); break;
        case 7: launch_attn_w<KT, HD, 7>(grid, s, q, kc, vc, n_q, n_kv, cap, scale, nsplit, po, pml, ctrl, w); break;
        case 8: launch_attn_w<KT, HD, 8>(grid, s, q, kc, vc, n_q, n_kv, cap, scale, nsplit, po, pml, ctrl, w); break;
        default: return vsl_unsupported("vsl_attn_decode: GQA ratio %u (supported 1..8)", G);
    }
    HIP_TRY(hipGetLastError());
    if (nsplit <= 32)
        k_attn_combine<HD, 32><<<n_q, kCombineThreads, 0, s>>>(po, pml, nsplit, out, ctrl);
    else if (nsplit <= (uint32_t)kFastSplits)
        k_attn_combine<HD, kFastSplits><<<n_q, kCombineThreads, 0, s>>>(po, pml, nsplit, out, ctrl);
    else
        k_attn_combine<HD, 0><<<n_q, kCombineThreads, 0, s>>>(po, pml, nsplit, out, ctrl);
    HIP_TRY(hipGetLastError());
    return VSL_OK;
}

// ---------------------------------------------------------------------------------------------
// samplers on logits in memory (top-k seeded, greedy) -- one block
// ---------------------------------------------------------------------------------------------
constexpr int kSampBlock = 1024;
constexpr int kMaxTopK = VSL_MAX_TOP_K;  // larger k (k = min(top_k, V)): VSL_E_UNSUPPORTED
constexpr int kWaveTopK = 64;            // k up to this: the threshold from per-thread maxima, weights one per lane
constexpr int kTauPerWave = 8;  // per-wave maxima entering the threshold: 16 waves x 8 = 128 keys
constexpr int kTopKChunks = kMaxTopK / kSampBlock;  // larger k: chunks of kSampBlock keys, one boundary each
static_assert(kSampBlock / 64 * kTauPerWave == 2 * VSL_WAVE && kWaveTopK <= VSL_WAVE, "threshold sort holds two keys per lane");
static_assert(kMaxTopK % kSampBlock == 0, "the selected keys are sorted one per thread, kSampBlock at a time");

__device__ __forceinline__ float sample_uniform(uint32_t k0, uint32_t k1, uint64_t step) {
    uint32_t c[4] = {(uint32_t)step, (uint32_t)(step >> 32), 0u, 0u};
    philox4x32_10(c, k0, k1);
    return (float)(c[0] >> 8) * (1.0f / 16777216.0f);
}

// Top-k order as a single unsigned key, larger = earlier: the high word orders the floats by value
// (-0 as +0, every NaN below -inf, where the reference's comparator has no order), the low word is
// the inverted index so that equal values put the lower index first.  No two elements share a key.
__device__ __forceinline__ uint32_t value_key(float v) {
    if (v != v) return 0u;
    uint32_t b = __float_as_uint(v);
    if (b == 0x80000000u) b = 0u;
    return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}
__device__ __forceinline__ float key_value(uint32_t k) {
    if (k == 0u) return __uint_as_float(0x7FC00000u);
    return __uint_as_float((k & 0x80000000u) ? (k & 0x7FFFFFFFu) : ~k);
}
__device__ __forceinline__ uint64_t rank_key(uint32_t vkey, uint32_t i) { return ((uint64_t)vkey << 32) | (uint32_t)~i; }
__device__ __forceinline__ uint64_t shfl_xor_u64(uint64_t v, int m) {
    const uint32_t lo = __shfl_xor((uint32_t)v, m, VSL_WAVE), hi = __shfl_xor((uint32_t)(v >> 32), m, VSL_WAVE);
    return ((uint64_t)hi << 32) | lo;
}

// Bitonic sort, descending, one key per thread of the first N threads: thread r ends holding the key
// of rank r.  Partners closer than a wave exchange through shuffles; farther ones through buf (N
// keys of LDS), so N > 64 needs every thread of the block, N = 64 one whole wave.
template <int N>
__device__ __forceinline__ uint64_t bitonic_desc(uint64_t x, uint32_t t, uint64_t* buf) {
#pragma unroll
    for (uint32_t size = 2; size <= (uint32_t)N; size <<= 1) {
#pragma unroll
        for (uint32_t stride = size >> 1; stride > 0; stride >>= 1) {
            uint64_t y;
            if (stride >= (uint32_t)VSL_WAVE) {
                buf[t] = x;
                __syncthreads();
                y = buf[t ^ stride];
                __syncthreads();
            } else {
                y = shfl_xor_u64(x, (int)stride);
            }
            const bool ascending_run = (t & size) != 0, lower = (t & stride) == 0;
            const uint64_t hi = x > y ? x : y, lo = x > y ? y : x;
            x = lower != ascending_run ? hi : lo;
        }
    }
    return x;
}

// Bitonic sort, descending, of 64 * M keys held by one wave, M per lane (key r of the sequence in
// register r / 64 of lane r % 64): rank r ends in the same place.  No LDS, no barriers.
template <int M>
__device__ __forceinline__ void wave_bitonic_desc(uint64_t (&x)[M], uint32_t lane) {
#pragma unroll
    for (uint32_t size = 2; size <= (uint32_t)(VSL_WAVE * M); size <<= 1) {
#pragma unroll
        for (uint32_t stride = size >> 1; stride > 0; stride >>= 1) {
            if (stride >= (uint32_t)VSL_WAVE) {
                const int rs = (int)(stride / VSL_WAVE);
#pragma unroll
                for (int m = 0; m < M; ++m) {
                    if (m & rs) continue;
                    const bool ascending_run = (((uint32_t)m * VSL_WAVE + lane) & size) != 0;
                    const uint64_t a = x[m], b = x[m | rs];
                    const uint64_t hi = a > b ? a : b, lo = a > b ? b : a;
                    x[m] = ascending_run ? lo : hi;
                    x[m | rs] = ascending_run ? hi : lo;
                }
            } else {
#pragma unroll
                for (int m = 0; m < M; ++m) {
                    const uint64_t y = shfl_xor_u64(x[m], (int)stride);
                    const bool ascending_run = (((uint32_t)m * VSL_WAVE + lane) & size) != 0;
                    const bool lower = (lane & stride) == 0;
                    const uint64_t hi = x[m] > y ? x[m] : y, lo = x[m] > y ? y : x[m];
                    x[m] = lower != ascending_run ? hi : lo;
                }
            }
        }
    }
}

// Calls f(v, base) for every batch of this thread's logits: v[j] is logit base + tid + j * kSampBlock
// (0 past V); the batch's loads are all issued before f runs.  One block streams at about 0.2
// cycles per logit whether or not the next batch is prefetched (the CU's outstanding misses bound
// it), so there is no prefetch.
constexpr int kSampBatch = 16;
template <class F>
__device__ __forceinline__ void for_each_logit_batch(const float* __restrict__ logits, uint32_t V, uint32_t tid, F&& f) {
    for (uint32_t base = 0; base < V; base += kSampBlock * kSampBatch) {
        float v[kSampBatch];
#pragma unroll
        for (int j = 0; j < kSampBatch; ++j) {
            const uint32_t i = base + tid + (uint32_t)j * kSampBlock;
            v[j] = i < V ? logits[i] : 0.f;
        }
        f(v, base);
    }
}

// Calls f(value, index) for every logit of this thread, in increasing index order.
template <class F>
__device__ __forceinline__ void for_each_logit(const float* __restrict__ logits, uint32_t V, uint32_t tid, F&& f) {
    for_each_logit_batch(logits, V, tid, [&](const float (&v)[kSampBatch], uint32_t base) {
#pragma unroll
        for (int j = 0; j < kSampBatch; ++j) {
            const uint32_t i = base + tid + (uint32_t)j * kSampBlock;
            if (i < V) f(v[j], i);
        }
    });
}

// The m-th largest rank key below ub (1 <= m <= the number of keys below ub): a most-significant-digit
// radix select over the 64-bit rank keys, 8 bits per pass, each pass streaming the logits and counting,
// in a 256-bin LDS histogram, the keys below ub that share the digits chosen so far.  The index half of
// the key is reached only when several logits share the boundary value and not all of them are taken;
// a pass whose chosen digit bin is taken whole ends the select (the boundary is then those digits with
// zeros below: the least key carrying them).
__device__ uint64_t select_below(const float* __restrict__ logits, uint32_t V, uint64_t ub, uint32_t m, uint32_t* hist) {
    __shared__ uint64_t s_pref;
    __shared__ uint32_t s_rem, s_full;
    const uint32_t tid = threadIdx.x;
    uint64_t prefix = 0, mask = 0;
    uint32_t remaining = m;  // how many of the keys matching `prefix` are still to be taken
    for (int pass = 0; pass < 8; ++pass) {
        const int shift = 56 - 8 * pass;
        if (tid < 256) hist[tid] = 0;
        __syncthreads();
        for_each_logit(logits, V, tid, [&](float l, uint32_t i) {
            const uint64_t e = rank_key(value_key(l), i);
            if (e < ub && (e & mask) == prefix) atomicAdd(&hist[(uint32_t)(e >> shift) & 255u], 1u);
        });
        __syncthreads();
        if (tid == 0) {
            // the digit holding the remaining-th largest key: the bins above it hold fewer keys
            uint32_t above = 0;
            int d = 255;
            for (; d > 0 && above + hist[d] < remaining; --d) above += hist[d];
            s_pref = prefix | ((uint64_t)d << shift);
            s_rem = remaining - above;
            s_full = hist[d] == remaining - above ? 1u : 0u;  // every key with these digits is taken
        }
        __syncthreads();
        prefix = s_pref;
        remaining = s_rem;
        mask |= (uint64_t)255u << shift;
        const bool full = s_full != 0u;
        __syncthreads();
        if (full) break;
    }
    return prefix;
}

// Gathers the m keys in [lo, ub) into cand and sorts them: rank r of the range in cand[r] (sorted:
// kSampBlock keys of LDS for the exchange).
__device__ void gather_sorted(const float* __restrict__ logits, uint32_t V, uint64_t lo, uint64_t ub, uint32_t m,
                              uint64_t* cand, uint64_t* sorted) {
    __shared__ uint32_t s_n;
    const uint32_t tid = threadIdx.x;
    if (tid == 0) s_n = 0;
    __syncthreads();
    for_each_logit(logits, V, tid, [&](float l, uint32_t i) {
        const uint64_t e = rank_key(value_key(l), i);
        if (e >= lo && e < ub) {
            const uint32_t slot = atomicAdd(&s_n, 1u);
            if (slot < (uint32_t)kSampBlock) cand[slot] = e;
        }
    });
    __syncthreads();
    uint64_t x = tid < m ? cand[tid] : 0ull;  // key 0 (a NaN at index 2^32 - 1) ranks below every key
    x = bitonic_desc<kSampBlock>(x, tid, sorted);
    if (tid < m) cand[tid] = x;
    __syncthreads();
}

// Seeded top-k for kWaveTopK < k <= kMaxTopK (Utils.cpp:151-171).  The k largest rank keys are taken in
// chunks of up to kSampBlock from the largest down: the chunk below ub (the previous chunk's last key;
// above every key at first) ends at the m-th largest key below ub (select_below), and its m keys are
// gathered and sorted by the block.  Rank keys are unique, so the chunks partition the top k exactly.
// The weights exp((l - max) / T) of a chunk are computed one per thread and added by one thread in rank
// order across the chunks (Utils.cpp:153-157); the walk then adds the weights w / sum in rank order
// chunk by chunk (:158-168), the chunks gathered again from their stored boundaries when there are
// several.  The arithmetic is that of the one-wave path, so both paths draw the same token from the
// same candidates.  cand and sorted hold kSampBlock keys of the caller's LDS.
__device__ uint32_t topk_sample_large(const float* __restrict__ logits, uint32_t V, uint32_t k, float temperature,
                                      uint32_t k0, uint32_t k1, uint64_t step, uint64_t* cand, uint64_t* sorted) {
    __shared__ uint32_t hist[256];
    __shared__ uint64_t s_lo[kTopKChunks];
    __shared__ float s_w[kSampBlock];
    __shared__ float s_sum;
    __shared__ uint32_t s_pick, s_found;
    const uint32_t tid = threadIdx.x;
    const uint32_t nch = (k + kSampBlock - 1) / kSampBlock;
    auto chunk_len = [&](uint32_t c) { return k - c * kSampBlock < (uint32_t)kSampBlock ? k - c * kSampBlock : (uint32_t)kSampBlock; };
    float mx = 0.f, sum = 0.f;  // sum: thread 0's running total
    uint64_t top = 0, ub = ~0ull;
    for (uint32_t c = 0; c < nch; ++c) {
        const uint32_t m = chunk_len(c);
        const uint64_t lo = select_below(logits, V, ub, m, hist);
        if (tid == 0) s_lo[c] = lo;
        gather_sorted(logits, V, lo, ub, m, cand, sorted);
        if (c == 0) {
            top = cand[0];
            mx = key_value((uint32_t)(top >> 32));
        }
        if (tid < m) s_w[tid] = expf((key_value((uint32_t)(cand[tid] >> 32)) - mx) / temperature);
        __syncthreads();
        if (tid == 0)
            for (uint32_t i = 0; i < m; ++i) sum += s_w[i];
        __syncthreads();
        ub = lo;
    }
    if (tid == 0) s_sum = sum;
    __syncthreads();
    sum = s_sum;
    const float r = sample_uniform(k0, k1, step);
    float cum = 0.f;  // thread 0's cumulative weight
    ub = ~0ull;
    for (uint32_t c = 0; c < nch; ++c) {
        const uint32_t m = chunk_len(c);
        if (nch > 1) gather_sorted(logits, V, s_lo[c], ub, m, cand, sorted);  // one chunk: still in cand
        if (tid < m) s_w[tid] = expf((key_value((uint32_t)(cand[tid] >> 32)) - mx) / temperature) / sum;
        __syncthreads();
        if (tid == 0) {
            s_found = 0u;
            for (uint32_t i = 0; i < m; ++i) {
                cum += s_w[i];
                if (r < cum) {
                    s_pick = ~(uint32_t)cand[i];
                    s_found = 1u;
                    break;
                }
            }
        }
        __syncthreads();
        const bool found = s_found != 0u;
        const uint32_t pick = s_pick;
        __syncthreads();
        if (found) return pick;
        ub = s_lo[c];
    }
    return ~(uint32_t)top;  // no cumulative weight passed r: the first element (Utils.cpp:169-170)
}

// Returns the sampled token (valid in every thread through LDS).  Every mode streams the logits
// from memory once per pass (the first pass brings them into the cache); nothing is held per
// element in registers.
__device__ __forceinline__ uint32_t block_sample(const float* __restrict__ logits, uint32_t V, int mode, float temperature,
                                 uint32_t top_k, uint32_t k0, uint32_t k1, uint64_t step) {
    __shared__ float wv[kSampBlock / 64];
    __shared__ uint32_t wi[kSampBlock / 64];
    __shared__ uint64_t s_sort[kSampBlock];
    __shared__ uint64_t s_cand[kSampBlock];
    __shared__ uint64_t s_top[kWaveTopK];
    __shared__ uint64_t s_best[kSampBlock / 64];
    __shared__ uint64_t s_tau;
    __shared__ uint32_t s_count;
    __shared__ uint32_t s_tok;
    const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    auto block_argmax = [&](float bv, uint32_t bi) -> uint32_t {  // first index of the max; none -> 0
        wave_argmax(bv, bi);
        if (lane == 0) { wv[wave] = bv; wi[wave] = bi; }
        __syncthreads();
        if (tid == 0) {
            float v = wv[0];
            uint32_t i = wi[0];
            for (int w = 1; w < kSampBlock / 64; ++w) argmax_merge(v, i, wv[w], wi[w]);
            s_tok = i == 0xFFFFFFFFu ? 0u : i;
        }
        __syncthreads();
        return s_tok;
    };
    if (mode == VSL_SAMPLE_GREEDY || temperature <= 0.f) {
        // greedy_sampling (VulkanSymbioteEngine.cpp:1794-1804): the first index of the largest logit,
        // over any V; a NaN first logit is never beaten, other NaNs never win.
        float bv = -INFINITY;
        uint32_t bi = 0xFFFFFFFFu;
        for_each_logit(logits, V, tid, [&](float l, uint32_t i) { argmax_merge(bv, bi, l, i); });
        const uint32_t tok = block_argmax(bv, bi);
        const float l0 = logits[0];
        return l0 != l0 ? 0u : tok;
    }
    if (mode == VSL_SAMPLE_REFERENCE) {
        // sample_token(T > 0) -> member top_k_sampling (VulkanSymbioteEngine.cpp:1806-1855) -> tokens[0]:
        // the first index of the largest fp32 probability exp(l/T - max) / sum.  That is the logit
        // argmax except where exp and the division round neighbours of the maximum to the same
        // probability; any NaN probability (a NaN or +inf logit) gives token 0, as there.
        __shared__ float red[kSampBlock / 64];
        auto scaled = [&](float l) { return temperature != 1.0f ? l / temperature : l; };
        float mx = -INFINITY;
        for_each_logit(logits, V, tid, [&](float l, uint32_t) { mx = fmaxf(mx, scaled(l)); });
        for (int o = 32; o >= 1; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o, VSL_WAVE));
        if (lane == 0) red[wave] = mx;
        __syncthreads();
        mx = red[0];
        for (int w = 1; w < kSampBlock / 64; ++w) mx = fmaxf(mx, red[w]);
        __syncthreads();
        float part = 0.f;
        for_each_logit(logits, V, tid, [&](float l, uint32_t) { part += expf(scaled(l) - mx); });
        for (int o = 32; o >= 1; o >>= 1) part += __shfl_xor(part, o, VSL_WAVE);
        if (lane == 0) red[wave] = part;
        __syncthreads();
        float sum = 0.f;
        for (int w = 0; w < kSampBlock / 64; ++w) sum += red[w];
        float bv = -INFINITY;
        uint32_t bi = 0xFFFFFFFFu;
        for_each_logit(logits, V, tid, [&](float l, uint32_t i) { argmax_merge(bv, bi, expf(scaled(l) - mx) / sum, i); });
        return block_argmax(bv, bi);
    }
    // Seeded top-k (Utils.cpp:151-171): the k first elements in rank-key order, exactly.  Every one
    // of them is >= tau whenever k distinct elements are >= tau; tau is the k-th largest of the
    // union of each wave's kTauPerWave largest per-thread maxima, so the elements >= tau -- about
    // k of them for ordinary logits -- hold the k and are sorted.  More than kSampBlock such
    // elements (many equal logits) take k rounds of "largest key below the last" instead.
    uint32_t k = top_k > V ? V : top_k;
    if (k > (uint32_t)kMaxTopK) k = kMaxTopK;  // refused by the launchers
    if (k > (uint32_t)kWaveTopK) return topk_sample_large(logits, V, k, temperature, k0, k1, step, s_cand, s_sort);
    float bf = -INFINITY;  // per-thread maximum, first index among equals; NaNs skipped
    uint32_t bi = 0xFFFFFFFFu;
    for_each_logit(logits, V, tid, [&](float l, uint32_t i) {
        if (l > bf || (bi == 0xFFFFFFFFu && l == l)) { bf = l; bi = i; }
    });
    uint64_t wm[1] = {bi == 0xFFFFFFFFu ? 0ull : rank_key(value_key(bf), bi)};  // 0 ranks below every element
    wave_bitonic_desc<1>(wm, lane);
    if (lane < (uint32_t)kTauPerWave) s_sort[wave * kTauPerWave + lane] = wm[0];
    if (tid == 0) s_count = 0;
    __syncthreads();
    if (wave == 0) {
        uint64_t u[2] = {s_sort[lane], s_sort[VSL_WAVE + lane]};
        wave_bitonic_desc<2>(u, lane);
        if (lane == k - 1) s_tau = u[0];  // k <= 64; tau = 0 when fewer than k threads hold a number
    }
    __syncthreads();
    const uint64_t tau = s_tau;
    const uint32_t tk = (uint32_t)(tau >> 32), ti = ~(uint32_t)tau;
    const float tf = key_value(tk);
    for_each_logit(logits, V, tid, [&](float l, uint32_t i) {
        // rank_key(value_key(l), i) >= tau in float compares (tk == 0: tau is a NaN or the sentinel)
        if (tk == 0u ? (l == l || i <= ti) : (l > tf || (l == tf && i <= ti))) {
            const uint32_t slot = atomicAdd(&s_count, 1u);
            if (slot < (uint32_t)kSampBlock) s_cand[slot] = rank_key(value_key(l), i);
        }
    });
    __syncthreads();
    const uint32_t total = s_count;
    if (total <= (uint32_t)VSL_WAVE) {
        if (wave == 0) {
            uint64_t x[1] = {lane < total ? s_cand[lane] : 0ull};
            wave_bitonic_desc<1>(x, lane);
            if (lane < k) s_top[lane] = x[0];
        }
    } else if (total <= 2u * VSL_WAVE) {
        if (wave == 0) {
            uint64_t x[2] = {s_cand[lane], VSL_WAVE + lane < total ? s_cand[VSL_WAVE + lane] : 0ull};
            wave_bitonic_desc<2>(x, lane);
            if (lane < k) s_top[lane] = x[0];
        }
    } else if (total <= (uint32_t)kSampBlock) {
        uint64_t x = tid < total ? s_cand[tid] : 0ull;
        x = bitonic_desc<kSampBlock>(x, tid, s_sort);
        if (tid < k) s_top[tid] = x;
    } else {
        uint64_t prev = ~0ull;
        for (uint32_t it = 0; it < k; ++it) {
            uint64_t best = 0;
            for_each_logit(logits, V, tid, [&](float l, uint32_t i) {
                const uint64_t e = rank_key(value_key(l), i);
                if (e < prev && e > best) best = e;
            });
#pragma unroll
            for (int o = 32; o >= 1; o >>= 1) {
                const uint64_t y = shfl_xor_u64(best, o);
                best = y > best ? y : best;
            }
            if (lane == 0) s_best[wave] = best;
            __syncthreads();
            prev = s_best[0];
            for (int w = 1; w < kSampBlock / 64; ++w) prev = s_best[w] > prev ? s_best[w] : prev;
            if (tid == 0) s_top[it] = prev;
            __syncthreads();
        }
    }
    __syncthreads();
    if (wave == 0) {
        // weights exp((l_i - max) / T) / sum in rank order: the sum and the cumulative walk in the
        // reference's sequential order (every lane of the wave computes the same sums)
        const uint64_t t = lane < k ? s_top[lane] : 0ull;
        const float mx = key_value((uint32_t)(s_top[0] >> 32));
        const float e = lane < k ? expf((key_value((uint32_t)(t >> 32)) - mx) / temperature) : 0.f;
        float sum = 0.f;
#pragma unroll
        for (int i = 0; i < kWaveTopK; ++i)
            if ((uint32_t)i < k) sum += __int_as_float(__builtin_amdgcn_readlane(__float_as_int(e), i));
        const int wi_bits = __float_as_int(e / sum);
        const float r = sample_uniform(k0, k1, step);
        float cum = 0.f;
        int pick = 0;
        bool found = false;
#pragma unroll
        for (int i = 0; i < kWaveTopK; ++i) {
            if ((uint32_t)i < k && !found) {
                cum += __int_as_float(__builtin_amdgcn_readlane(wi_bits, i));
                if (r < cum) { pick = i; found = true; }
            }
        }
        const uint32_t tok = ~(uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)t, pick);
        if (lane == 0) s_tok = tok;
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

// OM: output form, 0 plain (OT), 1 VSL_DT_F16X2, 2 VSL_DT_F16F8 (d % 32 == 0).
template <typename OT, int OM>
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
        if constexpr (OM == 1) {
            vsl_half hi, lo;
            split_f16(v, hi, lo);
            out[(size_t)blockIdx.x * d + i] = hi;
            out[(size_t)rows * d + (size_t)blockIdx.x * d + i] = lo;
        } else if constexpr (OM == 2) {
            vsl_half hi;
            uint32_t lo8;
            split_f16_f8(v, hi, lo8);
            out[(size_t)blockIdx.x * d + i] = hi;
            reinterpret_cast<uint8_t*>(out + (size_t)rows * d)[(size_t)blockIdx.x * d + lo8_pos(i)] = (uint8_t)lo8;
        } else {
            store_elem(out + (size_t)blockIdx.x * d + i, v);
        }
    }
}

// One row per wave, held in registers: NV float4 per lane (d = 256 NV), 16-byte loads of x and the
// gains, the sum of squares by DPP, 8-byte (fp16 / split) or 16-byte (fp32) stores. No LDS, no
// barrier: one memory round trip per row.
template <typename OT, int OM, int NV>
__global__ __launch_bounds__(kBlock) void k_rmsnorm_wave(const float* __restrict__ x, const float* __restrict__ gamma,
                                                         uint32_t rows, float eps, OT* __restrict__ out) {
    constexpr uint32_t d = 256 * NV;
    const uint32_t lane = threadIdx.x & 63;
    const uint32_t row = blockIdx.x * kWaves + (threadIdx.x >> 6);
    if (row >= rows) return;
    const float* xr = x + (size_t)row * d;
    float4 v[NV], g[NV];
#pragma unroll
    for (int j = 0; j < NV; ++j) v[j] = *reinterpret_cast<const float4*>(xr + (j * 64 + lane) * 4);
#pragma unroll
    for (int j = 0; j < NV; ++j)
        g[j] = gamma ? *reinterpret_cast<const float4*>(gamma + (j * 64 + lane) * 4) : make_float4(1.f, 1.f, 1.f, 1.f);
    float ss = 0.f;
#pragma unroll
    for (int j = 0; j < NV; ++j) ss += v[j].x * v[j].x + v[j].y * v[j].y + v[j].z * v[j].z + v[j].w * v[j].w;
    const float inv = 1.0f / sqrtf(wave_sum_dpp(ss) / (float)d + eps);
#pragma unroll
    for (int j = 0; j < NV; ++j) {
        const size_t o = (size_t)row * d + (j * 64 + lane) * 4;
        const float4 y = make_float4(v[j].x * inv * g[j].x, v[j].y * inv * g[j].y, v[j].z * inv * g[j].z,
                                     v[j].w * inv * g[j].w);
        if constexpr (OM == 1) {
            vsl_half h0, h1, h2, h3, l0, l1, l2, l3;
            split_f16(y.x, h0, l0);
            split_f16(y.y, h1, l1);
            split_f16(y.z, h2, l2);
            split_f16(y.w, h3, l3);
            *reinterpret_cast<half4*>(out + o) = half4{h0, h1, h2, h3};
            *reinterpret_cast<half4*>(out + (size_t)rows * d + o) = half4{l0, l1, l2, l3};
        } else if constexpr (OM == 2) {
            half4 h;
            uint32_t lo8;
            split4_f16_f8(y.x, y.y, y.z, y.w, h, lo8);
            *reinterpret_cast<half4*>(out + o) = h;
            const uint32_t c = (j * 64 + lane) * 4;
            *reinterpret_cast<uint32_t*>(reinterpret_cast<uint8_t*>(out + (size_t)rows * d) + (size_t)row * d +
                                         lo8_pos(c)) = lo8;
        } else if constexpr (sizeof(OT) == 2) {
            *reinterpret_cast<half4*>(out + o) = half4{(vsl_half)y.x, (vsl_half)y.y, (vsl_half)y.z, (vsl_half)y.w};
        } else {
            *reinterpret_cast<float4*>(out + o) = y;
        }
    }
}

template <typename OT, int X2>
void launch_rmsnorm(const float* x, const float* gamma, uint32_t rows, uint32_t d, float eps, OT* out, hipStream_t s) {
    const uint32_t wb = (rows + kWaves - 1) / kWaves;
    switch (d) {
        case 256: k_rmsnorm_wave<OT, X2, 1><<<wb, kBlock, 0, s>>>(x, gamma, rows, eps, out); return;
        case 512: k_rmsnorm_wave<OT, X2, 2><<<wb, kBlock, 0, s>>>(x, gamma, rows, eps, out); return;
        case 1024: k_rmsnorm_wave<OT, X2, 4><<<wb, kBlock, 0, s>>>(x, gamma, rows, eps, out); return;
        case 2048: k_rmsnorm_wave<OT, X2, 8><<<wb, kBlock, 0, s>>>(x, gamma, rows, eps, out); return;
        case 4096: k_rmsnorm_wave<OT, X2, 16><<<wb, kBlock, 0, s>>>(x, gamma, rows, eps, out); return;
        case 8192: k_rmsnorm_wave<OT, X2, 32><<<wb, kBlock, 0, s>>>(x, gamma, rows, eps, out); return;
        default: k_rmsnorm_rows<OT, X2><<<rows, kBlock, 0, s>>>(x, gamma, rows, d, eps, out); return;
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

// ---------------------------------------------------------------------------------------------
// skinny GEMM on MFMA (the fp16 GEMV sweep): Y[N][B] = W[N][K] X[K][B], X fp16 [K][B] row-major,
// 1 <= B <= 16, fp32 accumulation. v_mfma_f32_16x16x32_f16 with A = 16 rows of W (lane l: row
// l%16, k-slots 8*(l/16)..+7 -- one 16-byte load) and B = X (lane l: column l%16, the same
// k-slots -- eight 2-byte loads, L1/L2 resident); D lane l holds rows 4*(l/16)..+3 of column l%16.
// Block = kSkR x 16 rows x 8 waves (each wave's X operand serves its kSkR row groups); wave w
// accumulates the K range [w K/8, (w+1) K/8) in groups of U 32-wide steps, double-buffered (the next group's W loads issued before the current group's
// MFMAs); the 8 partial tiles are summed in LDS in wave order (deterministic). HBM traffic is W
// once; columns past B load column B-1 and are masked to zero.
// Block = kSkWaves waves splitting K, each wave kSkU k-steps of 32 per register group and R row
// tiles of 16 (R = 2 reuses each X fragment for two W tiles; chosen where N leaves enough blocks).
// W is read with ordinary (temporal) loads: a fragment load covers 64 bytes of each of 16 rows, and
// the next k-step's load the other half of those 128-byte lines, which then comes from L2. Measured
// on the sweep shapes (GB/s, geometric mean of the 12 points): 8 waves x 4 k-steps, non-temporal W
// 3564; 4 x 2 temporal 4218, with R = 2 for N >= 8192 and B >= 8 about 4350.
constexpr int kSkWaves = 4, kSkU = 2;
constexpr uint32_t kSkKAlign = kSkWaves * 32 * kSkU * 2;  // K multiple: whole group pairs per wave

// VEC_MAJOR: X holds B vectors of K ([B][K]) and Y B vectors of N ([B][N]) -- a batch of
// activation vectors, each contiguous -- so a lane's X operand is one 16-byte load; otherwise X is
// [K][B] and Y [N][B] (row-major products), eight 2-byte loads per operand.
template <typename YT, bool VEC_MAJOR, int R>
__global__ __launch_bounds__(kSkWaves * 64) void k_skinny(const vsl_half* __restrict__ W, uint32_t N, uint32_t K,
                                                         const vsl_half* __restrict__ X, uint32_t B, YT* __restrict__ Y) {
    constexpr uint32_t ROWS = 16 * R;  // rows per block
    __shared__ float part[kSkWaves][ROWS][17];
    const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const uint32_t row = blockIdx.x * ROWS + (lane & 15);  // + 16 per row tile
    const uint32_t ksub = (lane >> 4) * 8;
    const uint32_t col = lane & 15;
    const uint32_t bc = col < B ? col : B - 1;
    const uint32_t bmask = col < B ? 0xFFFFFFFFu : 0u;
    const uint32_t kw = K / kSkWaves;
    const uint32_t k_begin = wave * kw;
    const uint32_t n_groups = kw / (32 * kSkU);
    const vsl_half* wrow[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const uint32_t rr = row + 16 * r;
        wrow[r] = W + (size_t)(rr < N ? rr : N - 1) * K;  // rows past N: never stored
    }

    struct Group {
        uint4 a[R][kSkU];
        uint4 xv[kSkU];              // VEC_MAJOR
        vsl_half x[kSkU][VEC_MAJOR ? 1 : 8];
    };
    auto issue = [&](Group& g, uint32_t j) {
#pragma unroll
        for (int u = 0; u < kSkU; ++u) {
            const uint32_t k = k_begin + (j * kSkU + u) * 32 + ksub;
#pragma unroll
            for (int r = 0; r < R; ++r) g.a[r][u] = load16<false>(wrow[r] + k);
            if constexpr (VEC_MAJOR) {
                g.xv[u] = load16<false>(X + (size_t)bc * K + k);
            } else {
#pragma unroll
                for (int i = 0; i < 8; ++i) g.x[u][i] = X[(size_t)(k + i) * B + bc];
            }
        }
    };
    float4v acc[R];
#pragma unroll
    for (int r = 0; r < R; ++r) acc[r] = float4v{0.f, 0.f, 0.f, 0.f};
    auto consume = [&](const Group& g) {
#pragma unroll
        for (int u = 0; u < kSkU; ++u) {
            uint4 xr;
            if constexpr (VEC_MAJOR) {
                xr = g.xv[u];
            } else {
                half8 xb;
#pragma unroll
                for (int i = 0; i < 8; ++i) xb[i] = g.x[u][i];
                xr = __builtin_bit_cast(uint4, xb);
            }
            xr = make_uint4(xr.x & bmask, xr.y & bmask, xr.z & bmask, xr.w & bmask);
#pragma unroll
            for (int r = 0; r < R; ++r)
                acc[r] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8, g.a[r][u]),
                                                                __builtin_bit_cast(half8, xr), acc[r], 0, 0, 0);
        }
    };
    // n_groups is even (K % kSkKAlign == 0): the pair loop consumes exactly the wave's groups
    Group ga, gb;
    issue(ga, 0);
    for (uint32_t j = 0; j < n_groups; j += 2) {
        issue(gb, j + 1);
        __builtin_amdgcn_sched_barrier(0);
        consume(ga);
        issue(ga, j + 2 < n_groups ? j + 2 : j + 1);  // past the end: re-read, never consumed
        __builtin_amdgcn_sched_barrier(0);
        consume(gb);
    }
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int i = 0; i < 4; ++i) part[wave][16 * r + (lane >> 4) * 4 + i][col] = acc[r][i];
    __syncthreads();
    for (uint32_t e = threadIdx.x; e < ROWS * 16; e += kSkWaves * 64) {
        const uint32_t m = e >> 4, n = e & 15;
        float v = 0.f;
#pragma unroll
        for (int w = 0; w < kSkWaves; ++w) v += part[w][m][n];
        const uint32_t r = blockIdx.x * ROWS + m;
        if (r < N && n < B) store_elem(Y + (VEC_MAJOR ? (size_t)n * N + r : (size_t)r * B + n), v);
    }
}

// The same product with both operands staged through LDS (X [B][K], K % 1024 == 0): block = 16 rows x
// 4 waves splitting K, each wave its own double-buffered LDS chunks of 128 columns -- the 16 W rows
// and the 16 X vectors (vectors past B re-read vector B-1 and are masked). Every load instruction
// (global_load_lds) moves 256-byte runs of four rows, whole 128-byte lines, where the register
// fragment loads of k_skinny take 64 bytes of each of 16 rows; the fragments come from LDS, chunk q
// of row r stored at position q ^ r so that the 16 rows of a fragment read fall in distinct banks.
// Each wave waits only for its own copies (vmcnt): no block barrier until the partial tiles are summed
// in wave order. 64 KB of LDS per block, two blocks per CU. Sweep at B = 16 (GB/s, geometric mean of
// the four shapes): k_skinny 3690; chunks of 256 columns (one block per CU) 4160, 128 x 4 buffers 4155,
// 128 x 2 buffers 4500, 64 x 2 4180, 64 x 4 4336, 128 x 2 with 8 waves 4187.
constexpr int kSlWaves = 4;
template <uint32_t CH_, int NB_>
struct SlCfg {
    static constexpr uint32_t CH = CH_;  // columns of K per LDS chunk
    static constexpr int NB = NB_;       // chunk buffers per wave (NB - 1 in flight)
    static constexpr uint32_t RUN = CH * 2;             // bytes of one row per chunk
    static constexpr uint32_t LPR = RUN / 16;           // lanes per row in a load instruction
    static constexpr uint32_t RPI = 64 / LPR;           // rows per load instruction
    static constexpr uint32_t NLD = 16 / RPI;           // load instructions per operand and chunk
    static constexpr uint32_t KALIGN = kSlWaves * CH * NB;
    static_assert(LPR <= 64 && 16 % RPI == 0 && LPR >= 8, "rows of 128 .. 1024 bytes per chunk");
    // position of logical 16-byte chunk q of row r: the 16 rows of a fragment read in distinct bank
    // groups (a 256-byte LDS cycle holds one row of 256+ bytes, or two rows of 128)
    static __device__ __forceinline__ uint32_t pos(uint32_t q, uint32_t r) {
        return LPR >= 16 ? q ^ (r & 15) : q ^ ((r >> 1) & 7);
    }
};
using SlDefault = SlCfg<128, 2>;
constexpr uint32_t kSlKAlign = SlDefault::KALIGN;  // K multiple: whole buffer rounds per wave
static_assert(SlDefault::KALIGN % SlCfg<64, 2>::KALIGN == 0, "the row-group variants take the same K");
constexpr uint32_t kSlRowsFor4 = 25600, kSlRowsFor2 = 12800;  // N from which 4 / 2 row groups per block

template <class C, typename YT>
__global__ __launch_bounds__(kSlWaves * 64) void k_skinny_lds(const vsl_half* __restrict__ W, uint32_t N, uint32_t K,
                                                             const vsl_half* __restrict__ X, uint32_t B,
                                                             YT* __restrict__ Y) {
    constexpr uint32_t CH = C::CH, REG = 16 * CH;  // halfs per operand region (16 rows / vectors)
    constexpr int NB = C::NB;
    __shared__ __attribute__((aligned(16))) vsl_half buf[kSlWaves][NB][2 * REG];  // [wave][buffer][W | X]
    __shared__ float part[kSlWaves][16][17];
    const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const uint32_t row0 = blockIdx.x * 16;
    const uint32_t kw = K / kSlWaves, k_begin = wave * kw, nch = kw / CH;
    // load instruction j covers rows / vectors RPI j .. RPI j + RPI - 1 (LPR lanes each); lane position
    // p of its row holds logical chunk p ^ (row & 15)
    const uint32_t p = lane % C::LPR, rsub = lane / C::LPR;
    uint32_t woff[C::NLD], xoff[C::NLD];
#pragma unroll
    for (int j = 0; j < (int)C::NLD; ++j) {
        const uint32_t rr = C::RPI * j + rsub;
        const uint32_t wrow = row0 + rr < N ? row0 + rr : N - 1;  // rows past N: never stored
        const uint32_t xcol = rr < B ? rr : B - 1;                // vectors past B: masked
        woff[j] = (wrow * K + k_begin + C::pos(p, rr) * 8) * 2;  // pos is its own inverse
        xoff[j] = (xcol * K + k_begin + C::pos(p, rr) * 8) * 2;
    }
    auto issue = [&](uint32_t c, int bsel) {
        const uint32_t cc = c < nch ? c : nch - 1;  // past the end: re-load the last chunk (never read)
        vsl_half* L = buf[wave][bsel];
#pragma unroll
        for (int j = 0; j < (int)C::NLD; ++j) lds_load16(W + cc * CH, woff[j], L + j * 512);
#pragma unroll
        for (int j = 0; j < (int)C::NLD; ++j) lds_load16(X + cc * CH, xoff[j], L + REG + j * 512);
    };
    const uint32_t r = lane & 15, g = lane >> 4;
    const uint32_t bmask = r < B ? 0xFFFFFFFFu : 0u;  // this lane's X fragment is vector r
    float4v acc = float4v{0.f, 0.f, 0.f, 0.f};
    auto consume = [&](int bsel) {
        const vsl_half* L = buf[wave][bsel];
#pragma unroll
        for (int u = 0; u < (int)(CH / 32); ++u) {
            const uint32_t pos = C::pos(4 * u + g, r) * 8;
            const half8 a = *reinterpret_cast<const half8*>(L + r * CH + pos);
            uint4 xv = __builtin_bit_cast(uint4, *reinterpret_cast<const half8*>(L + REG + r * CH + pos));
            xv = make_uint4(xv.x & bmask, xv.y & bmask, xv.z & bmask, xv.w & bmask);
            acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, __builtin_bit_cast(half8, xv), acc, 0, 0, 0);
        }
    };
    // chunk c in buffer c % NB; chunks c + 1 .. c + NB - 1 in flight while c is consumed; nch % NB == 0
    constexpr int kPer = 2 * C::NLD;  // loads per chunk
#pragma unroll
    for (int b = 0; b < NB - 1; ++b) issue(b, b);
    for (uint32_t c = 0; c < nch; c += NB) {
#pragma unroll
        for (int b = 0; b < NB; ++b) {
            issue(c + b + NB - 1, (b + NB - 1) % NB);
            VSL_VMCNT_WAIT((NB - 1) * kPer);
            consume(b);
            VSL_LGKM_WAIT0();  // buffer b fully read before it is refilled
        }
    }
    VSL_VMCNT_WAIT(0);  // the trailing re-loads land before the LDS is released
#pragma unroll
    for (int i = 0; i < 4; ++i) part[wave][(lane >> 4) * 4 + i][r] = acc[i];
    __syncthreads();
    for (uint32_t e = threadIdx.x; e < 16 * 16; e += kSlWaves * 64) {
        const uint32_t m = e >> 4, n = e & 15;
        float v = 0.f;
#pragma unroll
        for (int w = 0; w < kSlWaves; ++w) v += part[w][m][n];
        const uint32_t row = row0 + m;
        if (row < N && n < B) store_elem(Y + (size_t)n * N + row, v);
    }
}

// The same with RB 16-row groups of W per block sharing every staged X chunk (X crosses L2 -> LDS once
// per RB x 16 rows instead of once per 16); each wave's partial tile goes through its own buffers.
template <class C, int RB, typename YT>
__global__ __launch_bounds__(kSlWaves * 64) void k_skinny_lds_rg(const vsl_half* __restrict__ W, uint32_t N, uint32_t K,
                                                             const vsl_half* __restrict__ X, uint32_t B,
                                                             YT* __restrict__ Y) {
    constexpr uint32_t CH = C::CH, REGX = 16 * CH, REGW = RB * REGX;  // halfs per operand region
    constexpr int NB = C::NB;
    constexpr uint32_t NLDW = RB * C::NLD;  // W load instructions per chunk
    constexpr uint32_t PSTRIDE = 17;        // floats per row of a wave's partial tile (padded)
    static_assert((REGW + REGX) * 2 * NB >= 16 * RB * PSTRIDE * 4, "partials fit in a wave's buffers");
    __shared__ __attribute__((aligned(16))) vsl_half buf[kSlWaves][NB][REGW + REGX];  // [wave][buffer][W | X]
    const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const uint32_t row0 = blockIdx.x * 16 * RB;
    const uint32_t kw = K / kSlWaves, k_begin = wave * kw, nch = kw / CH;
    // load instruction j covers rows / vectors RPI j .. RPI j + RPI - 1 (LPR lanes each); lane position
    // p of its row holds logical chunk pos(p, row) (the swizzle is its own inverse)
    const uint32_t p = lane % C::LPR, rsub = lane / C::LPR;
    uint32_t woff[NLDW], xoff[C::NLD];
#pragma unroll
    for (int j = 0; j < (int)NLDW; ++j) {
        const uint32_t rr = C::RPI * j + rsub;
        const uint32_t wrow = row0 + rr < N ? row0 + rr : N - 1;  // rows past N: never stored
        woff[j] = (wrow * K + k_begin + C::pos(p, rr) * 8) * 2;
    }
#pragma unroll
    for (int j = 0; j < (int)C::NLD; ++j) {
        const uint32_t rr = C::RPI * j + rsub;
        const uint32_t xcol = rr < B ? rr : B - 1;  // vectors past B: masked
        xoff[j] = (xcol * K + k_begin + C::pos(p, rr) * 8) * 2;
    }
    auto issue = [&](uint32_t c, int bsel) {
        const uint32_t cc = c < nch ? c : nch - 1;  // past the end: re-load the last chunk (never read)
        vsl_half* L = buf[wave][bsel];
#pragma unroll
        for (int j = 0; j < (int)NLDW; ++j) lds_load16(W + cc * CH, woff[j], L + j * 512);
#pragma unroll
        for (int j = 0; j < (int)C::NLD; ++j) lds_load16(X + cc * CH, xoff[j], L + REGW + j * 512);
    };
    const uint32_t r = lane & 15, g = lane >> 4;
    const uint32_t bmask = r < B ? 0xFFFFFFFFu : 0u;  // this lane's X fragment is vector r
    float4v acc[RB];
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) acc[rb] = float4v{0.f, 0.f, 0.f, 0.f};
    auto consume = [&](int bsel) {
        const vsl_half* L = buf[wave][bsel];
#pragma unroll
        for (int u = 0; u < (int)(CH / 32); ++u) {
            const uint32_t pos = C::pos(4 * u + g, r) * 8;  // rows 16 rb + r share the swizzle of row r
            uint4 xv = __builtin_bit_cast(uint4, *reinterpret_cast<const half8*>(L + REGW + r * CH + pos));
            xv = make_uint4(xv.x & bmask, xv.y & bmask, xv.z & bmask, xv.w & bmask);
            const half8 xf = __builtin_bit_cast(half8, xv);
#pragma unroll
            for (int rb = 0; rb < RB; ++rb) {
                const half8 a = *reinterpret_cast<const half8*>(L + (rb * 16 + r) * CH + pos);
                acc[rb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, xf, acc[rb], 0, 0, 0);
            }
        }
    };
    // chunk c in buffer c % NB; chunks c + 1 .. c + NB - 1 in flight while c is consumed; nch % NB == 0
    constexpr int kPer = NLDW + C::NLD;  // loads per chunk
#pragma unroll
    for (int b = 0; b < NB - 1; ++b) issue(b, b);
    for (uint32_t c = 0; c < nch; c += NB) {
#pragma unroll
        for (int b = 0; b < NB; ++b) {
            issue(c + b + NB - 1, (b + NB - 1) % NB);
            VSL_VMCNT_WAIT((NB - 1) * kPer);
            consume(b);
            VSL_LGKM_WAIT0();  // buffer b fully read before it is refilled
        }
    }
    VSL_VMCNT_WAIT(0);  // the trailing re-loads land before the buffers take the partials
    // each wave's partial tile goes into its own (now idle) buffers; summed over the waves in order
    float* part = reinterpret_cast<float*>(&buf[wave][0][0]);
#pragma unroll
    for (int rb = 0; rb < RB; ++rb)
#pragma unroll
        for (int i = 0; i < 4; ++i) part[(rb * 16 + (lane >> 4) * 4 + i) * PSTRIDE + r] = acc[rb][i];
    __syncthreads();
    for (uint32_t e = threadIdx.x; e < 16 * 16 * RB; e += kSlWaves * 64) {
        const uint32_t m = e >> 4, n = e & 15;
        float v = 0.f;
#pragma unroll
        for (int w = 0; w < kSlWaves; ++w) v += reinterpret_cast<const float*>(&buf[w][0][0])[m * PSTRIDE + n];
        const uint32_t row = row0 + m;
        if (row < N && n < B) store_elem(Y + (size_t)n * N + row, v);
    }
}

template <typename YT, bool VEC_MAJOR>
int launch_skinny(const void* W, uint32_t N, uint32_t K, const void* X, uint32_t B, void* Y, hipStream_t s) {
    const vsl_half* w = static_cast<const vsl_half*>(W);
    const vsl_half* x = static_cast<const vsl_half*>(X);
    if (N >= 8192 && B >= 8)
        k_skinny<YT, VEC_MAJOR, 2><<<(N + 31) / 32, kSkWaves * 64, 0, s>>>(w, N, K, x, B, static_cast<YT*>(Y));
    else
        k_skinny<YT, VEC_MAJOR, 1><<<(N + 15) / 16, kSkWaves * 64, 0, s>>>(w, N, K, x, B, static_cast<YT*>(Y));
    HIP_TRY(hipGetLastError());
    return VSL_OK;
}

// Small-batch GEMV (2 <= B <= 8, X fp16 [B][K] staged once per block in LDS): whole rows per wave as
// in the decode GEMV, every weight load a 1 KB-contiguous run of one row (64 lanes x 16 bytes), two
// tiles of R rows in flight per wave; each 16-byte weight chunk meets the same 8 elements of every
// vector through v_dot2_f32_f16 (two fp16 products -- exact in fp32 -- added to an fp32 accumulator),
// and the R rows of a wave share every activation read. One 16-wave block per CU; per-lane partial
// sums reduced by DPP at the end of each row group.
constexpr int kRowsWaves = 16;
constexpr uint32_t kRowsLdsBytes = 128u << 10;  // X of at most B * K * 2 bytes

__device__ __forceinline__ float dot8(uint4 w, uint4 x, float acc) {
    acc = __builtin_amdgcn_fdot2(__builtin_bit_cast(half2v, w.x), __builtin_bit_cast(half2v, x.x), acc, false);
    acc = __builtin_amdgcn_fdot2(__builtin_bit_cast(half2v, w.y), __builtin_bit_cast(half2v, x.y), acc, false);
    acc = __builtin_amdgcn_fdot2(__builtin_bit_cast(half2v, w.z), __builtin_bit_cast(half2v, x.z), acc, false);
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(half2v, w.w), __builtin_bit_cast(half2v, x.w), acc, false);
}

// K % 1024 == 0 (an even number of 512-wide tiles: the tile pairs below never load past a row). A
// wave requests its first group's first two tiles before the block stages X, and the next group's
// first two tiles before it reduces and stores the current group, so the weight stream never waits
// on the staging or the reductions.
template <int B, int R, class YT>
__global__ __launch_bounds__(kRowsWaves * 64) void k_gemv_rows(const vsl_half* __restrict__ W, uint32_t N, uint32_t K,
                                                             const vsl_half* __restrict__ X, YT* __restrict__ Y) {
    extern __shared__ uint4 xrows[];  // X [B][K], 8 halfs per entry
    constexpr uint32_t NT = kRowsWaves * 64;
    const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const uint32_t kq = K / 8, tiles = K / 512;
    const uint32_t groups = (N + R - 1) / R, gstride = gridDim.x * kRowsWaves;
    const vsl_half* wr[R];
    auto set_rows = [&](uint32_t g) {  // rows past N (and groups past the last) read row N - 1
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const uint32_t row = g * R + r;
            wr[r] = W + (size_t)(row < N ? row : N - 1) * K + lane * 8;
        }
    };
    uint4 ta[R], tb[R];
    auto load = [&](uint4 (&t)[R], uint32_t tile) {
#pragma unroll
        for (int r = 0; r < R; ++r) t[r] = load16<true>(wr[r] + (size_t)tile * 512);
    };
    uint32_t g = blockIdx.x * kRowsWaves + wave;
    set_rows(g);
    load(ta, 0);
    load(tb, 1);
    for (uint32_t i = tid; i < (uint32_t)B * kq; i += NT) xrows[i] = load16<false>(X + (size_t)i * 8);
    __syncthreads();
    for (; g < groups; g += gstride) {
        float acc[R][B];
#pragma unroll
        for (int r = 0; r < R; ++r)
#pragma unroll
            for (int b = 0; b < B; ++b) acc[r][b] = 0.f;
        auto use = [&](const uint4 (&t)[R], uint32_t tile) {
            // one address register per tile, each vector's (uniform) offset added in the loop: left to
            // itself the compiler keeps a strength-reduced address per vector and buffer live
            uint32_t off = (tile * 64 + lane) * 16;
            asm volatile("" : "+v"(off));
            const char* xb = reinterpret_cast<const char*>(xrows) + off;
#pragma unroll
            for (int b = 0; b < B; ++b) {
                const uint4 xv = *reinterpret_cast<const uint4*>(xb + (size_t)b * kq * 16);
#pragma unroll
                for (int r = 0; r < R; ++r) acc[r][b] = dot8(t[r], xv, acc[r][b]);
            }
        };
        for (uint32_t t = 0; t + 2 < tiles; t += 2) {
            use(ta, t);
            load(ta, t + 2);
            use(tb, t + 1);
            load(tb, t + 3);
        }
        const uint32_t g0 = g;
        set_rows(g + gstride);  // the next group (its tiles are requested even past the last group)
        use(ta, tiles - 2);
        load(ta, 0);
        use(tb, tiles - 1);
        load(tb, 1);
#pragma unroll
        for (int r = 0; r < R; ++r)
#pragma unroll
            for (int b = 0; b < B; ++b) {
                const float v = wave_sum_dpp(acc[r][b]);
                const uint32_t row = g0 * R + r;
                if (lane == 0 && row < N) Y[(size_t)b * N + row] = (YT)v;
            }
    }
}

template <int B, int R, class YT>
int launch_rows_br(const vsl_half* w, uint32_t N, uint32_t K, const vsl_half* x, YT* y, hipStream_t s) {
    const size_t lds = (size_t)B * K * 2;
    static bool attr = false;
    if (!attr) {
        HIP_TRY(hipFuncSetAttribute(reinterpret_cast<const void*>(&k_gemv_rows<B, R, YT>),
                                    hipFuncAttributeMaxDynamicSharedMemorySize, (int)kRowsLdsBytes));
        attr = true;
    }
    uint32_t blocks = ((N + R - 1) / R + kRowsWaves - 1) / kRowsWaves;
    const uint32_t cap = gemv_grid_cap(kRowsWaves, EPI_STORE);
    if (blocks > cap) blocks = cap;
    k_gemv_rows<B, R, YT><<<blocks, kRowsWaves * 64, lds, s>>>(w, N, K, x, y);
    HIP_TRY(hipGetLastError());
    return VSL_OK;
}

// One row per wave (sweep B = 4, interleaved runs: geometric mean 5053-5075 GB/s, against 4560 with
// two rows per wave sharing each activation read from 8192 rows on -- 14336 rows in pairs leave the
// 4096 waves one or two groups each -- and 4110 for the MFMA kernel).
template <int B, class YT>
int launch_rows_b(const vsl_half* w, uint32_t N, uint32_t K, const vsl_half* x, YT* y, hipStream_t s) {
    return launch_rows_br<B, 1>(w, N, K, x, y, s);
}

// Whether k_gemv_rows serves a batched product: 2 <= B <= 8, X (B * K * 2 bytes) fits the block's
// LDS, K % 1024 == 0 and X 16-byte aligned.  At B = 16 the 16 activation reads and 64 dot2 per 1 KB
// of weights bound it at 1.1-1.8 TB/s on the sweep shapes, against 3.5-3.9 for the MFMA kernel.
bool rows_fits(uint32_t B, uint32_t K, const void* X) {
    return B >= 2 && B <= 8 && (uint64_t)B * K * 2 <= kRowsLdsBytes && K % 1024 == 0 &&
           (reinterpret_cast<uintptr_t>(X) & 15) == 0;
}

template <class YT>
int launch_rows(const void* W, uint32_t N, uint32_t K, const void* X, uint32_t B, void* Y, hipStream_t s) {
    const vsl_half* w = static_cast<const vsl_half*>(W);
    const vsl_half* x = static_cast<const vsl_half*>(X);
    YT* y = static_cast<YT*>(Y);
    switch (B) {
        case 2: return launch_rows_b<2>(w, N, K, x, y, s);
        case 3: return launch_rows_b<3>(w, N, K, x, y, s);
        case 4: return launch_rows_b<4>(w, N, K, x, y, s);
        case 5: return launch_rows_b<5>(w, N, K, x, y, s);
        case 6: return launch_rows_b<6>(w, N, K, x, y, s);
        case 7: return launch_rows_b<7>(w, N, K, x, y, s);
        case 8: return launch_rows_b<8>(w, N, K, x, y, s);
        default: return vsl_invalid("k_gemv_rows: B=%u", B);
    }
}

}  // namespace

// One fp16 activation vector against fp16 W: the decode GEMV (whole rows per wave, two rows per tile,
// the vector staged in LDS as fp32), which streams W faster than the MFMA sweep kernel at B = 1.
static int gemv_one_f16x(const void* W, uint32_t N, uint32_t K, const void* X, void* Y, int ydtype, hipStream_t s) {
    if (int rc = check_gemv_shape(N, K, "vsl_gemv (B = 1)")) return rc;
    GemvArgs a{};
    a.W = W;
    a.N = N;
    a.K = K;
    a.xh = static_cast<const vsl_half*>(X);
    a.y = static_cast<float*>(Y);
    // one row per wave for short W (twice the waves in flight: 4096 x 4096 4.0 -> 4.6 TB/s), two above
    if (N <= 8192)
        return ydtype == VSL_DT_F16 ? launch_gemv_k<WF16, 1, 4, EPI_STORE_F16>(a, 1u << 20, s)
                                    : launch_gemv_k<WF16, 1, 4, EPI_STORE>(a, 1u << 20, s);
    return ydtype == VSL_DT_F16 ? launch_gemv_k<WF16, 2, 4, EPI_STORE_F16>(a, 1u << 20, s)
                                : launch_gemv_k<WF16, 2, 4, EPI_STORE>(a, 1u << 20, s);
}

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
    if (out_dtype == VSL_DT_F16F8 && d % 32) return vsl_invalid("vsl_rmsnorm: F16F8 needs d %% 32 == 0 (d = %u)", d);
    if (out_dtype == VSL_DT_F16)
        launch_rmsnorm<vsl_half, 0>(x, gamma, rows, d, eps, static_cast<vsl_half*>(out), s);
    else if (out_dtype == VSL_DT_F16X2)
        launch_rmsnorm<vsl_half, 1>(x, gamma, rows, d, eps, static_cast<vsl_half*>(out), s);
    else if (out_dtype == VSL_DT_F16F8)
        launch_rmsnorm<vsl_half, 2>(x, gamma, rows, d, eps, static_cast<vsl_half*>(out), s);
    else if (out_dtype == VSL_DT_F32)
        launch_rmsnorm<float, 0>(x, gamma, rows, d, eps, static_cast<float*>(out), s);
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
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (quant_dtype(wdtype) && B == 1 && xdtype == VSL_DT_F32 && (ydtype == VSL_DT_F16 || ydtype == VSL_DT_F32)) {
        // a block-quantized pack: the decode GEMV (B = 1, fp32 X)
        GemvArgs a{};
        a.W = W;
        a.N = N;
        a.K = K;
        a.x = static_cast<const float*>(X);
        a.y = static_cast<float*>(Y);
        return ydtype == VSL_DT_F16 ? launch_gemv_w<2, EPI_STORE_F16>(wdtype, a, 1u << 20, s, "vsl_gemv")
                                    : launch_gemv_w<2, EPI_STORE>(wdtype, a, 1u << 20, s, "vsl_gemv");
    }
    if ((wdtype != VSL_DT_F16 && wdtype != VSL_DT_F32) || (xdtype != VSL_DT_F16 && xdtype != VSL_DT_F32) ||
        (ydtype != VSL_DT_F16 && ydtype != VSL_DT_F32))
        return vsl_unsupported("vsl_gemv: dtype combination %d/%d/%d", wdtype, xdtype, ydtype);
    if (wdtype == VSL_DT_F16 && xdtype == VSL_DT_F16 && B == 1 && K % 8 == 0 && K <= kMaxK &&
        (reinterpret_cast<uintptr_t>(X) & 7) == 0)
        return gemv_one_f16x(W, N, K, X, Y, ydtype, s);
    if (wdtype == VSL_DT_F16 && xdtype == VSL_DT_F16 && K % kSkKAlign == 0)
        return ydtype == VSL_DT_F16 ? launch_skinny<vsl_half, false>(W, N, K, X, B, Y, s)
                                    : launch_skinny<float, false>(W, N, K, X, B, Y, s);
    if (B == 1) {
        if (xdtype == VSL_DT_F16)
            return vsl_unsupported("vsl_gemv: B=1 with fp16 X needs K %% %u == 0 (else pass fp32 X)", kSkKAlign);
        GemvArgs a{};
        a.W = W;
        a.N = N;
        a.K = K;
        a.x = static_cast<const float*>(X);
        a.y = static_cast<float*>(Y);
        if (wdtype == VSL_DT_F16)
            return ydtype == VSL_DT_F16 ? launch_gemv_k<WF16, 2, 4, EPI_STORE_F16>(a, 1u << 20, s)
                                        : launch_gemv_k<WF16, 2, 4, EPI_STORE>(a, 1u << 20, s);
        return ydtype == VSL_DT_F16 ? launch_gemv_k<WF32, 2, 4, EPI_STORE_F16>(a, 1u << 20, s)
                                    : launch_gemv_k<WF32, 2, 4, EPI_STORE>(a, 1u << 20, s);
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

extern "C" int vsl_gemv_batched(const void* W, uint32_t N, uint32_t K, const void* X, uint32_t B, void* Y, int ydtype,
                                void* stream) {
    if (!W || !X || !Y) return vsl_invalid("vsl_gemv_batched: null pointer");
    if (N == 0 || K == 0) return vsl_invalid("vsl_gemv_batched: empty shape");
    if (B < 1 || B > 16) return vsl_invalid("vsl_gemv_batched: B=%u must be in [1,16]", B);
    if (K % kSkKAlign) return vsl_invalid("vsl_gemv_batched: K=%u must be a multiple of %u", K, kSkKAlign);
    if (ydtype != VSL_DT_F16 && ydtype != VSL_DT_F32) return vsl_unsupported("vsl_gemv_batched: Y dtype %d", ydtype);
    hipStream_t s = static_cast<hipStream_t>(stream);
    // the decode GEMV stages X with 8-byte loads; an X that is only 2-byte aligned takes the MFMA kernel
    if (B == 1 && K <= kMaxK && (reinterpret_cast<uintptr_t>(X) & 7) == 0) return gemv_one_f16x(W, N, K, X, Y, ydtype, s);
    if (rows_fits(B, K, X))
        return ydtype == VSL_DT_F16 ? launch_rows<vsl_half>(W, N, K, X, B, Y, s) : launch_rows<float>(W, N, K, X, B, Y, s);
    if (K % kSlKAlign == 0 && (reinterpret_cast<uintptr_t>(X) & 15) == 0 && ((uint64_t)N * K * 2) >> 32 == 0 &&
        ((uint64_t)B * K * 2) >> 32 == 0) {
        const vsl_half* w = static_cast<const vsl_half*>(W);
        const vsl_half* x = static_cast<const vsl_half*>(X);
        auto go = [&](auto rbc) {
            using C = SlCfg<64, 2>;
            constexpr int RB = decltype(rbc)::value;
            const uint32_t grid = (N + 16 * RB - 1) / (16 * RB);
            if (ydtype == VSL_DT_F16)
                k_skinny_lds_rg<C, RB, vsl_half><<<grid, kSlWaves * 64, 0, s>>>(w, N, K, x, B, static_cast<vsl_half*>(Y));
            else
                k_skinny_lds_rg<C, RB, float><<<grid, kSlWaves * 64, 0, s>>>(w, N, K, x, B, static_cast<float*>(Y));
        };
        // tall W: several 16-row groups per block share each staged X chunk, as long as the grid keeps
        // about two blocks per CU
        if (N >= kSlRowsFor4) go(std::integral_constant<int, 4>{});
        else if (N >= kSlRowsFor2) go(std::integral_constant<int, 2>{});
        else if (ydtype == VSL_DT_F16)
            k_skinny_lds<SlDefault, vsl_half><<<(N + 15) / 16, kSlWaves * 64, 0, s>>>(w, N, K, x, B, static_cast<vsl_half*>(Y));
        else
            k_skinny_lds<SlDefault, float><<<(N + 15) / 16, kSlWaves * 64, 0, s>>>(w, N, K, x, B, static_cast<float*>(Y));
        HIP_TRY(hipGetLastError());
        return VSL_OK;
    }
    return ydtype == VSL_DT_F16 ? launch_skinny<vsl_half, true>(W, N, K, X, B, Y, s)
                                : launch_skinny<float, true>(W, N, K, X, B, Y, s);
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
    if (kv_dtype == VSL_DT_F16) return launch_gemv_w<2, EPI_QKV, WF16>(wdtype, a, 1u << 20, s, "vsl_qkv_rope_append");
    return launch_gemv_w<2, EPI_QKV, WF32>(wdtype, a, 1u << 20, s, "vsl_qkv_rope_append");
}

static int attn_decode(const float* q, const void* kcache, const void* vcache, int kv_dtype, uint32_t n_q,
                       uint32_t n_kv, uint32_t hd, uint32_t cap, float scale, uint32_t nsplit, float* part_o,
                       float* part_ml, float* out, vsl_ctrl* ctrl, const AttnWindow& w, void* stream) {
    if (!q || !kcache || !vcache || !part_o || !part_ml || !out || !ctrl)
        return vsl_invalid("vsl_attn_decode: null pointer");
    if (n_kv == 0 || n_q % n_kv) return vsl_invalid("vsl_attn_decode: n_q=%u not a multiple of n_kv=%u", n_q, n_kv);
    if (nsplit == 0 || nsplit > kMaxSplits) return vsl_invalid("vsl_attn_decode: nsplit=%u (1..%u)", nsplit, kMaxSplits);
    const uint32_t G = n_q / n_kv;
    dim3 grid(nsplit, n_kv);
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (kv_dtype == VSL_DT_F16) {
        if (hd == 128) return launch_attn_g<WF16, 128>(G, grid, s, q, kcache, vcache, n_q, n_kv, cap, scale, nsplit, part_o, part_ml, out, ctrl, w);
        if (hd == 64) return launch_attn_g<WF16, 64>(G, grid, s, q, kcache, vcache, n_q, n_kv, cap, scale, nsplit, part_o, part_ml, out, ctrl, w);
    } else if (kv_dtype == VSL_DT_F32) {
        if (hd == 128) return launch_attn_g<WF32, 128>(G, grid, s, q, kcache, vcache, n_q, n_kv, cap, scale, nsplit, part_o, part_ml, out, ctrl, w);
        if (hd == 64) return launch_attn_g<WF32, 64>(G, grid, s, q, kcache, vcache, n_q, n_kv, cap, scale, nsplit, part_o, part_ml, out, ctrl, w);
    }
    return vsl_unsupported("vsl_attn_decode: head_dim %u / kv dtype %d (supported 64,128 / f16,f32)", hd, kv_dtype);
}

extern "C" int vsl_attn_decode(const float* q, const void* kcache, const void* vcache, int kv_dtype, uint32_t n_q,
                               uint32_t n_kv, uint32_t hd, uint32_t cap, float scale, uint32_t nsplit, float* part_o,
                               float* part_ml, float* out, vsl_ctrl* ctrl, void* stream) {
    return attn_decode(q, kcache, vcache, kv_dtype, n_q, n_kv, hd, cap, scale, nsplit, part_o, part_ml, out, ctrl,
                       AttnWindow{false, 0, 0, 0}, stream);
}

extern "C" int vsl_attn_decode_window(const float* q, const void* kcache, const void* vcache, int kv_dtype,
                                      uint32_t n_q, uint32_t n_kv, uint32_t hd, uint32_t cap, float scale,
                                      uint32_t nsplit, float* part_o, float* part_ml, float* out, vsl_ctrl* ctrl,
                                      uint32_t window, uint32_t n_global, uint32_t threshold, void* stream) {
    if ((uint64_t)window + n_global >= 0x80000000ull)
        return vsl_invalid("vsl_attn_decode_window: window %u + global %u too large", window, n_global);
    return attn_decode(q, kcache, vcache, kv_dtype, n_q, n_kv, hd, cap, scale, nsplit, part_o, part_ml, out, ctrl,
                       AttnWindow{true, window, n_global, threshold}, stream);
}

// ---------------------------------------------------------------------------------------------
// vsl_attn_decode without a caller workspace: the split partials live in a static device array.
// ---------------------------------------------------------------------------------------------
// Up to kScratchPairs (query head, split) pairs of partials: an fp32 output row of up to
// kScratchHd dims each, then the (m, l) pairs.  2 MiB + 32 KiB per GPU, held until the process ends.
constexpr uint32_t kScratchPairs = 4096, kScratchHd = 128;
constexpr size_t kScratchFloats = (size_t)kScratchPairs * (kScratchHd + 2);
static __device__ __align__(256) float scratch[kScratchFloats];

// The array's address on the current device, looked up once per device (each GPU holds its own copy;
// the array's name in host code is not a device address).  nullptr after a failed lookup.
static float* scratch_on_current_device() {
    constexpr int kMaxDevices = 64;
    static std::mutex mu;
    static float* addr[kMaxDevices] = {};
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) {
        vsl_set_error("vsl_attn_decode_noalloc: no current device (or device id >= %d)", kMaxDevices);
        return nullptr;
    }
    std::lock_guard<std::mutex> lk(mu);
    if (!addr[dev]) {
        void* p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p) {
            vsl_set_error("vsl_attn_decode_noalloc: hipGetSymbolAddress(scratch) on device %d: %s", dev,
                          hipGetErrorString(e));
            return nullptr;
        }
        addr[dev] = static_cast<float*>(p);
    }
    return addr[dev];
}

extern "C" int vsl_attn_decode_noalloc(const float* q, const void* kcache, const void* vcache, int kv_dtype,
                                       uint32_t n_q, uint32_t n_kv, uint32_t hd, uint32_t cap, float scale,
                                       uint32_t nsplit, float* out, vsl_ctrl* ctrl, void* stream) {
    if ((uint64_t)n_q * nsplit > kScratchPairs || hd > kScratchHd)
        return vsl_capacity("vsl_attn_decode_noalloc: n_q * nsplit = %llu (max %u) and head_dim %u (max %u) "
                            "exceed the static partials buffer",
                            (unsigned long long)n_q * nsplit, kScratchPairs, hd, kScratchHd);
    float* base = scratch_on_current_device();
    if (!base) return VSL_E_HIP;
    // same layout as a caller workspace: part_o [n_q][nsplit][hd], then part_ml [n_q][nsplit][2]
    float* part_o = base;
    float* part_ml = base + (size_t)kScratchPairs * kScratchHd;
    return attn_decode(q, kcache, vcache, kv_dtype, n_q, n_kv, hd, cap, scale, nsplit, part_o, part_ml, out, ctrl,
                       AttnWindow{false, 0, 0, 0}, stream);
}

extern "C" int vsl_gemv_residual(const void* W, int wdtype, uint32_t N, uint32_t K, const float* x, float* resid,
                                 vsl_ctrl* ctrl, void* stream) {
    if (!W || !x || !resid) return vsl_invalid("vsl_gemv_residual: null pointer");
    if (int rc = check_gemv_shape(N, K, "vsl_gemv_residual")) return rc;
    GemvArgs a{};
    a.W = W; a.N = N; a.K = K; a.x = x; a.y = resid; a.ctrl = ctrl;
    hipStream_t s = static_cast<hipStream_t>(stream);
    return launch_gemv_w<1, EPI_RESID>(wdtype, a, 1u << 20, s, "vsl_gemv_residual");
}

extern "C" int vsl_norm_swiglu(const float* x, const float* gamma, float eps, const void* Wgu, int wdtype, uint32_t d,
                               uint32_t F, float* h_out, vsl_ctrl* ctrl, void* stream) {
    if (!x || !Wgu || !h_out) return vsl_invalid("vsl_norm_swiglu: null pointer");
    if (int rc = check_gemv_shape(F, d, "vsl_norm_swiglu")) return rc;
    GemvArgs a{};
    a.W = Wgu; a.N = F; a.K = d; a.x = x; a.gamma = gamma; a.eps = eps; a.y = h_out; a.ctrl = ctrl;
    hipStream_t s = static_cast<hipStream_t>(stream);
    return launch_gemv_w<2, EPI_SWIGLU>(wdtype, a, 1u << 20, s, "vsl_norm_swiglu");
}

extern "C" uint32_t vsl_lm_head_ws_blocks(void) { return kMaxLmBlocks; }

// Sampler arguments the kernels serve: a known mode, and for seeded top-k 1 <= min(top_k, V) <=
// kMaxTopK (top_k > V means all of V).
static int check_sampler(const vsl_sampler& sp, uint32_t V, const char* who) {
    if (sp.mode < VSL_SAMPLE_GREEDY || sp.mode > VSL_SAMPLE_TOPK_SEEDED) return vsl_invalid("%s: sampler mode %d", who, sp.mode);
    if (sp.temperature <= 0.f || sp.mode == VSL_SAMPLE_GREEDY) return VSL_OK;  // greedy: no limits
    const uint32_t k = sp.top_k < V ? sp.top_k : V;
    if (sp.mode == VSL_SAMPLE_TOPK_SEEDED && (sp.top_k == 0 || k > (uint32_t)kMaxTopK))
        return vsl_unsupported("%s: seeded top-k supports 1 <= min(top_k, V) <= %d (got top_k %u, V %u)", who,
                               kMaxTopK, sp.top_k, V);
    return VSL_OK;
}

extern "C" int vsl_lm_head_sample(const float* gamma, float eps, const void* W, int wdtype, uint32_t V, uint32_t d,
                                  float* x, const void* embed, int embed_dtype, float* logits, vsl_sampler sampler,
                                  float* ws_val, uint32_t* ws_idx, uint32_t* tokens, vsl_ctrl* ctrl, void* stream) {
    if (!W || !x || !embed || !logits || !ws_val || !ws_idx || !tokens || !ctrl)
        return vsl_invalid("vsl_lm_head_sample: null pointer");
    if (int rc = check_gemv_shape(V, d, "vsl_lm_head_sample")) return rc;
    if (embed_dtype != VSL_DT_F16 && embed_dtype != VSL_DT_F32) return vsl_unsupported("embed dtype %d", embed_dtype);
    if (wdtype != VSL_DT_F16 && wdtype != VSL_DT_F32 && !quant_dtype(wdtype))
        return vsl_unsupported("vsl_lm_head_sample: dtype %d", wdtype);
    if (quant_dtype(wdtype) && d % 32) return vsl_invalid("vsl_lm_head_sample: a block-quantized pack needs d %% 32 == 0");
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (int rc = check_sampler(sampler, V, "vsl_lm_head_sample")) return rc;
    const bool fused = sampler.mode == VSL_SAMPLE_GREEDY || sampler.temperature <= 0.f;
    GemvArgs a{};
    a.W = W; a.N = V; a.K = d; a.x = x; a.gamma = gamma; a.eps = eps; a.y = logits;
    a.ws_val = ws_val; a.ws_idx = ws_idx; a.tokens = tokens; a.embed = embed; a.x_next = x;
    a.ctrl = ctrl;
    if (fused) {
        int rc = launch_gemv_w<2, EPI_ARGMAX>(wdtype, a, kMaxLmBlocks, s, "vsl_lm_head_sample");
        if (rc) return rc;
        const uint32_t nb = gemv_blocks_k<2, EPI_ARGMAX>(V, d, kMaxLmBlocks);
        if (embed_dtype == VSL_DT_F16)
            k_argmax_finish<WF16><<<1, kFinishThreads, 0, s>>>(ws_val, ws_idx, nb, V, d, embed, x, tokens, ctrl);
        else
            k_argmax_finish<WF32><<<1, kFinishThreads, 0, s>>>(ws_val, ws_idx, nb, V, d, embed, x, tokens, ctrl);
        HIP_TRY(hipGetLastError());
        return VSL_OK;
    }
    // logits only (EPI_STORE with the norm prologue), then the sampling kernel
    int rc = launch_gemv_w<2, EPI_STORE>(wdtype, a, 1u << 20, s, "vsl_lm_head_sample");
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
    if (int rc = check_sampler(sampler, V, "vsl_sample_logits")) return rc;
    const uint64_t key = vsl_derive_key(sampler.seed, "sampler");
    k_sample_logits<<<1, kSampBlock, 0, static_cast<hipStream_t>(stream)>>>(
        logits, V, sampler.mode, sampler.temperature, sampler.top_k, (uint32_t)key, (uint32_t)(key >> 32), step, out);
    HIP_TRY(hipGetLastError());
    return VSL_OK;
}
