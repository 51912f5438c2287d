// vsl_prefill.hip -- prefill (S positions at once) on gfx950 MFMA.
//
// k_gemm_f16:      C[M][N] = A[M][K] * B[N][K]^T with v_mfma_f32_32x32x16_f16, 128x128 block tile,
//                  BK = 32, LDS double buffering, fused epilogues (fp32 / fp16 store, residual add,
//                  SwiGLU over [Wgate; Wup]).
// k_rope_split:    QKV GEMM output -> RoPE(q, k) at positions pos0+s -> q (fp16), K/V cache (fp16).
// k_attn_prefill:  causal flash attention, one block per (32 query rows, KV head) with one wave per
//                  query head of the group, computing S^T = K Q^T and O^T = V^T P^T on MFMA so that
//                  every lane owns one query row's softmax statistics and output column.
//
// MFMA 32x32x16 f16 operand layout used here (lane l of a 64-lane wave):
//   A (32 x 16): row l%32, 8 consecutive k-slots 8*(l/32)..+7
//   B (16 x 32): col l%32, the same 8 k-slots
//   D (32 x 32): 16 floats; element v is row (v/4)*8 + (l/32)*4 + v%4, col l%32
// Which physical k a slot holds is free as long as A and B agree.
#include <hip/hip_runtime.h>

#include <type_traits>

#include <cmath>

#include "vsl_device.h"
#include "vsl_hip.h"
#include "vsl_internal.h"

namespace {

constexpr int BK = 64;  // K per pipeline stage
constexpr int CH = 8;   // halfs per 16-byte chunk; a tile row holds BK / CH = 8 chunks

// Tile configurations: block BM x BN, WAVES_M x WAVES_N waves, each wave a (BM/WAVES_M) x
// (BN/WAVES_N) sub-tile of 32x32 MFMA fragments.
//   GemmBig   128 x 256, 2 x 2 waves of 64 x 128 (8 accumulators per wave: long independent MFMA
//             chains, 0.5 KB of LDS reads per MFMA) -- the wide projections;
//   GemmMid   128 x 128, 4 x 2 waves of 32 x 64 (two waves per SIMD);
//   GemmSmall  64 x 128, 2 x 2 waves of 32 x 64 (twice the tiles when the others leave CUs idle).
template <int BM_, int BN_, int WAVES_M_, int WAVES_N_>
struct GemmCfg {
    static constexpr int BM = BM_, BN = BN_, WAVES_M = WAVES_M_, WAVES_N = WAVES_N_;
    static constexpr int NT = 64 * WAVES_M * WAVES_N;
    static constexpr int WM = BM / WAVES_M, WN = BN / WAVES_N, FM = WM / 32, FN = WN / 32;
};
using GemmBig = GemmCfg<128, 256, 2, 2>;
using GemmMid = GemmCfg<128, 128, 4, 2>;
using GemmSmall = GemmCfg<64, 128, 2, 2>;

__device__ __forceinline__ int d_row(int v, int lane) { return (v >> 2) * 8 + (lane >> 5) * 4 + (v & 3); }

// LDS tiles are unpadded rows of BK halfs (128 bytes). gfx950's LDS serves 256 bytes (64 banks)
// per cycle, i.e. 16 lanes of a 16-byte access: two rows. The 16-byte chunk c of row r is stored at
// chunk position c ^ ((r >> 1) & 7): a fragment read (16 consecutive lanes = 16 consecutive rows,
// one logical chunk) then covers all 16 bank groups (row parity x 8 positions), and so does a
// store of two whole rows. No bank conflicts, no padding.
__device__ __forceinline__ int swz(int r, int c) { return r * BK + ((c ^ ((r >> 1) & 7)) * CH); }

// Block tile -> (m-tile, n-tile). Workgroups are dispatched to the 8 XCDs round-robin by block id;
// each XCD gets a contiguous range of tiles, m-tiles fastest, so the blocks sharing a weight tile
// share that XCD's L2. Returns false for the idle tail blocks of the last XCD ranges.
__device__ __forceinline__ bool tile_of(uint32_t n_m, uint32_t n_tiles, uint32_t& mt, uint32_t& nt) {
    const uint32_t b = blockIdx.x, xcd = b & 7, slot = b >> 3;
    const uint32_t per = (n_tiles + 7) >> 3;
    const uint32_t t = xcd * per + slot;
    if (slot >= per || t >= n_tiles) return false;
    mt = t % n_m;
    nt = t / n_m;
    return true;
}

// C[M][N] = A[M][K] * B[N][K]^T for one tile configuration (GemmCfg). Per K stage of 64: A (both
// planes when split) and B tiles go global -> registers -> LDS (double buffered); each stage's
// global loads are issued two stages ahead of its LDS stores.
template <class G, int EPI, bool AX2, bool CX2>
__global__ __launch_bounds__(G::NT) void k_gemm_f16(const vsl_half* __restrict__ A, const vsl_half* __restrict__ B,
                                                    uint32_t M, uint32_t N, uint32_t K, void* __restrict__ C) {
    constexpr int BM = G::BM, BN = G::BN, NT = G::NT, WM = G::WM, WN = G::WN, FM = G::FM, FN = G::FN;
    constexpr int AP = AX2 ? 2 : 1;  // A planes (hi, lo)
    constexpr int ACH = BM * BK / CH / NT;  // A chunks per thread per plane
    constexpr int BCH = BN * BK / CH / NT;  // B chunks per thread
    static_assert(EPI != VSL_EPI_SWIGLU || FN % 2 == 0, "SwiGLU waves pair gate and up fragments");
    __shared__ __attribute__((aligned(16))) vsl_half As[2][AP][BM * BK];
    __shared__ __attribute__((aligned(16))) vsl_half Bs[2][BN * BK];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave / G::WAVES_N, wn = wave % G::WAVES_N;
    const uint32_t ncols = EPI == VSL_EPI_SWIGLU ? BN / 2 : BN;
    const uint32_t n_m = (M + BM - 1) / BM, n_n = N / ncols;
    uint32_t mt, nt;
    if (!tile_of(n_m, n_m * n_n, mt, nt)) return;
    const uint32_t m0 = mt * BM;
    // EPI_SWIGLU: the block covers 64 output columns; B-tile rows 0..63 are gate rows, 64..127 up rows.
    const uint32_t nout0 = nt * ncols;
    const size_t plane = (size_t)M * K;

    auto b_row = [&](int r) -> uint32_t {
        if constexpr (EPI == VSL_EPI_SWIGLU) return r < BN / 2 ? nout0 + r : N + nout0 + (r - BN / 2);
        else return nout0 + r;
    };
    // Rows past M load row M-1 (never stored). K need only be a multiple of 32: chunks past K load
    // chunk 0 of their row and are zeroed when stored to LDS (the mask is applied there, not at the
    // load, so no select waits on a load in flight).
    struct Stage {
        uint4 a[AP][ACH], b[BCH];
    };
    auto gload = [&](Stage& st, uint32_t k0) {
#pragma unroll
        for (int i = 0; i < ACH; ++i) {
            const int c = tid + i * NT, r = c >> 3, ck = c & 7;
            const uint32_t gr = m0 + r < M ? m0 + r : M - 1;
            const uint32_t kk = k0 + ck * CH;
#pragma unroll
            for (int p = 0; p < AP; ++p)
                st.a[p][i] = *reinterpret_cast<const uint4*>(A + p * plane + (size_t)gr * K + (kk < K ? kk : 0));
        }
#pragma unroll
        for (int i = 0; i < BCH; ++i) {
            const int c = tid + i * NT, r = c >> 3, ck = c & 7;
            const uint32_t kk = k0 + ck * CH;
            st.b[i] = *reinterpret_cast<const uint4*>(B + (size_t)b_row(r) * K + (kk < K ? kk : 0));
        }
    };
    // (masking by AND on the values: a select between the register set and a zero constant would
    // be lowered as a select of addresses and keep the sets out of registers)
    auto masked = [](uint4 v, uint32_t m) { return make_uint4(v.x & m, v.y & m, v.z & m, v.w & m); };
    auto sstore = [&](const Stage& st, int buf, uint32_t k0) {
#pragma unroll
        for (int i = 0; i < ACH; ++i) {
            const int c = tid + i * NT, r = c >> 3, ck = c & 7;
            const uint32_t m = k0 + ck * CH < K ? 0xFFFFFFFFu : 0u;
#pragma unroll
            for (int p = 0; p < AP; ++p) *reinterpret_cast<uint4*>(&As[buf][p][swz(r, ck)]) = masked(st.a[p][i], m);
        }
#pragma unroll
        for (int i = 0; i < BCH; ++i) {
            const int c = tid + i * NT, r = c >> 3, ck = c & 7;
            const uint32_t m = k0 + ck * CH < K ? 0xFFFFFFFFu : 0u;
            *reinterpret_cast<uint4*>(&Bs[buf][swz(r, ck)]) = masked(st.b[i], m);
        }
    };

    float16v acc[FM][FN];
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j)
#pragma unroll
            for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.f;

    // B-tile rows of this wave's FN 32-column fragments; for SwiGLU the first FN/2 are gate rows
    // and the last FN/2 the matching up rows
    int bt[FN];
#pragma unroll
    for (int j = 0; j < FN; ++j) {
        if constexpr (EPI == VSL_EPI_SWIGLU)
            bt[j] = (j < FN / 2 ? 0 : BN / 2) + wn * (WN / 2) + (j % (FN / 2)) * 32;
        else
            bt[j] = wn * WN + j * 32;
    }

    // Fragments of k-step ks+1 are read from LDS before the MFMAs of k-step ks are issued.
    struct Frags {
        half8 a[AP][FM], b[FN];
    };
    auto fload = [&](Frags& f, int buf, int ks) {
        const int lc = ks * 2 + (lane >> 5);  // logical chunk of this lane's 8 k-slots
#pragma unroll
        for (int i = 0; i < FM; ++i) {
            const int r = wm * WM + i * 32 + (lane & 31);
#pragma unroll
            for (int p = 0; p < AP; ++p) f.a[p][i] = *reinterpret_cast<const half8*>(&As[buf][p][swz(r, lc)]);
        }
#pragma unroll
        for (int j = 0; j < FN; ++j) f.b[j] = *reinterpret_cast<const half8*>(&Bs[buf][swz(bt[j] + (lane & 31), lc)]);
    };
    auto mfmas = [&](const Frags& f) {
#pragma unroll
        for (int p = 0; p < AP; ++p)
#pragma unroll
            for (int i = 0; i < FM; ++i)
#pragma unroll
                for (int j = 0; j < FN; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(f.a[p][i], f.b[j], acc[i][j], 0, 0, 0);
    };
    // One stage = four 16-wide k-steps; the next k-step's fragments are read before the current
    // k-step's MFMAs are issued.
    static_assert(BK == 64, "compute() walks four 16-wide k-steps");
    auto compute = [&](int buf) {
        Frags f0, f1;
        fload(f0, buf, 0);
        fload(f1, buf, 1);
        mfmas(f0);
        fload(f0, buf, 2);
        mfmas(f1);
        fload(f1, buf, 3);
        mfmas(f0);
        mfmas(f1);
    };

    // Pipeline: stage k's global loads are issued two stages before it is stored to LDS (register
    // sets s0/s1 alternate), so each load has two stages of MFMA work to arrive. The stage count is
    // rounded up to even (a padding stage is all zeros); loads for stages past the end re-read the
    // last stage and are never stored, keeping every load unconditional.
    const uint32_t nk = ((K + 2 * BK - 1) / (2 * BK)) * 2;
    const uint32_t klast = (nk - 1) * BK;
    auto kof = [&](uint32_t st) { return st < nk ? st * BK : klast; };
    Stage s0, s1;
    gload(s0, 0);
    gload(s1, kof(1));
    sstore(s0, 0, 0);
    __syncthreads();
    for (uint32_t kt = 0; kt < nk; kt += 2) {
        gload(s0, kof(kt + 2));
        __builtin_amdgcn_sched_barrier(0);
        compute(0);
        sstore(s1, 1, (kt + 1) * BK);
        __syncthreads();
        gload(s1, kof(kt + 3));
        __builtin_amdgcn_sched_barrier(0);
        compute(1);
        sstore(s0, 0, (kt + 2) * BK);  // past the end: zeros, never read
        __syncthreads();
    }

    // epilogue
#pragma unroll
    for (int i = 0; i < FM; ++i) {
#pragma unroll
        for (int v = 0; v < 16; ++v) {
            const uint32_t row = m0 + wm * WM + i * 32 + d_row(v, lane);
            if (row >= M) continue;
            if constexpr (EPI == VSL_EPI_SWIGLU) {
                vsl_half* Ch = reinterpret_cast<vsl_half*>(C);
#pragma unroll
                for (int j = 0; j < FN / 2; ++j) {
                    const uint32_t col = nout0 + wn * (WN / 2) + j * 32 + (lane & 31);
                    const float h = silu(acc[i][j][v]) * acc[i][j + FN / 2][v];
                    if constexpr (CX2) {
                        vsl_half hi, lo;
                        split_f16(h, hi, lo);
                        Ch[(size_t)row * N + col] = hi;
                        Ch[(size_t)M * N + (size_t)row * N + col] = lo;
                    } else {
                        Ch[(size_t)row * N + col] = (vsl_half)h;
                    }
                }
            } else {
#pragma unroll
                for (int j = 0; j < FN; ++j) {
                    const uint32_t col = nout0 + wn * WN + j * 32 + (lane & 31);
                    const size_t o = (size_t)row * N + col;
                    if constexpr (EPI == VSL_EPI_STORE_F32) reinterpret_cast<float*>(C)[o] = acc[i][j][v];
                    else if constexpr (EPI == VSL_EPI_STORE_F16) reinterpret_cast<vsl_half*>(C)[o] = (vsl_half)acc[i][j][v];
                    else reinterpret_cast<float*>(C)[o] += acc[i][j][v];
                }
            }
        }
    }
}

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

// The same over four consecutive columns (two rotation pairs) per thread, with the projection given
// as KS fp32 k-chunk partials ws[KS][S][W] summed in chunk order (KS = 1: the finished projection):
// 16-byte loads of each partial, 8-byte loads of the rotation tables, 8-byte q and fp16 cache stores
// (16-byte fp32 cache stores). Needs hd % 4 == 0; a quad then never straddles a head or the q/k/v
// boundaries. KS = 0: the partial count is ks_rt, summed in the same order by a loop.
template <class KT, bool QX2, int KS>
__global__ __launch_bounds__(256) void k_rope_split4(const float* __restrict__ ws, uint32_t S, uint32_t n_q,
                                                     uint32_t n_kv, uint32_t hd, uint32_t pos0,
                                                     const float* __restrict__ rc, const float* __restrict__ rs,
                                                     vsl_half* __restrict__ q_out, void* __restrict__ kc,
                                                     void* __restrict__ vc, uint32_t cap, uint32_t ks_rt) {
    const uint32_t width = (n_q + 2 * n_kv) * hd, quads = width / 4;
    const uint64_t e = (uint64_t)blockIdx.x * 256 + threadIdx.x;
    if (e >= (uint64_t)S * quads) return;
    const uint32_t s = (uint32_t)(e / quads), col = (uint32_t)(e % quads) * 4;
    const uint64_t MN = (uint64_t)S * width;
    const size_t off = (size_t)s * width + col;
    float4v v = *reinterpret_cast<const float4v*>(ws + off);
    if constexpr (KS > 0) {
#pragma unroll
        for (int k = 1; k < KS; ++k) v += *reinterpret_cast<const float4v*>(ws + k * MN + off);
    } else {
#pragma unroll 8  // eight chunks' loads in flight, summed in order
        for (uint32_t k = 1; k < ks_rt; ++k) v += *reinterpret_cast<const float4v*>(ws + k * MN + off);
    }
    const uint32_t pos = pos0 + s, qw = n_q * hd, kw = n_kv * hd;
    if (col < qw + kw) {
        const size_t j = (size_t)pos * (hd >> 1) + ((col % hd) >> 1);
        const float2 c = *reinterpret_cast<const float2*>(rc + j);
        const float2 sn = *reinterpret_cast<const float2*>(rs + j);
        v = float4v{v[0] * c.x - v[1] * sn.x, v[0] * sn.x + v[1] * c.x, v[2] * c.y - v[3] * sn.y,
                    v[2] * sn.y + v[3] * c.y};
    }
    if (col < qw) {
        const size_t o = (size_t)s * qw + col;
        if constexpr (QX2) {
            vsl_half h0, h1, h2, h3, l0, l1, l2, l3;
            split_f16(v[0], h0, l0);
            split_f16(v[1], h1, l1);
            split_f16(v[2], h2, l2);
            split_f16(v[3], h3, l3);
            *reinterpret_cast<half4*>(q_out + o) = half4{h0, h1, h2, h3};
            *reinterpret_cast<half4*>(q_out + (size_t)S * qw + o) = half4{l0, l1, l2, l3};
        } else {
            *reinterpret_cast<half4*>(q_out + o) = half4{(vsl_half)v[0], (vsl_half)v[1], (vsl_half)v[2], (vsl_half)v[3]};
        }
    } else {
        typedef typename KT::T T;
        const bool is_k = col < qw + kw;
        const uint32_t cc = col - (is_k ? qw : qw + kw);
        T* dst = static_cast<T*>(is_k ? kc : vc) + ((size_t)(cc / hd) * cap + pos) * hd + cc % hd;
        if constexpr (sizeof(T) == 2)
            *reinterpret_cast<half4*>(dst) = half4{(vsl_half)v[0], (vsl_half)v[1], (vsl_half)v[2], (vsl_half)v[3]};
        else
            *reinterpret_cast<float4v*>(dst) = v;
    }
}

// Residual projection given as KS fp32 k-chunk partials ws[KS][rows][d]: x += their sum (chunks in
// order, then added to x), followed by the next RMSNorm of the updated rows, out = x / sqrt(mean(x^2)
// + eps) * gamma (OM: 0 fp16 or fp32 as OT, 1 VSL_DT_F16X2, 2 VSL_DT_F16F8). One 256-thread block per row, NV float4 per thread
// (d = 1024 NV): every partial, x and gamma requested before the first is used, x written once, the
// row's sum of squares by DPP within each wave and four floats of LDS across the waves. KS = 0: the
// partial count is ks_rt, summed in the same order by a loop (many partials: no register copy of each).
template <typename OT, int OM, int NV, int KS>
__global__ __launch_bounds__(256) void k_splitk_resid_rmsnorm(const float* __restrict__ ws, uint32_t rows,
                                                              float* __restrict__ x, const float* __restrict__ gamma,
                                                              float eps, OT* __restrict__ out, uint32_t ks_rt) {
    constexpr uint32_t d = 1024 * NV;
    __shared__ float red[4];
    const uint32_t t = threadIdx.x;
    const size_t base = (size_t)blockIdx.x * d;
    const uint64_t MN = (uint64_t)rows * d;
    float4v v[NV], g[NV];
#pragma unroll
    for (int j = 0; j < NV; ++j) v[j] = *reinterpret_cast<const float4v*>(ws + base + (j * 256 + t) * 4);
    if constexpr (KS > 0) {
#pragma unroll
        for (int k = 1; k < KS; ++k)
#pragma unroll
            for (int j = 0; j < NV; ++j) v[j] += *reinterpret_cast<const float4v*>(ws + k * MN + base + (j * 256 + t) * 4);
    } else {
        // unrolled so that eight chunks' loads are in flight at once (the sums stay in chunk order)
#pragma unroll 8
        for (uint32_t k = 1; k < ks_rt; ++k)
#pragma unroll
            for (int j = 0; j < NV; ++j) v[j] += *reinterpret_cast<const float4v*>(ws + k * MN + base + (j * 256 + t) * 4);
    }
#pragma unroll
    for (int j = 0; j < NV; ++j)
        g[j] = gamma ? *reinterpret_cast<const float4v*>(gamma + (j * 256 + t) * 4) : float4v{1.f, 1.f, 1.f, 1.f};
    float ss = 0.f;
#pragma unroll
    for (int j = 0; j < NV; ++j) {
        float4v* xp = reinterpret_cast<float4v*>(x + base + (j * 256 + t) * 4);
        v[j] = *xp + v[j];
        *xp = v[j];
        ss += v[j][0] * v[j][0] + v[j][1] * v[j][1] + v[j][2] * v[j][2] + v[j][3] * v[j][3];
    }
    ss = wave_sum_dpp(ss);
    if ((t & 63) == 0) red[t >> 6] = ss;
    __syncthreads();
    const float inv = 1.0f / sqrtf(((red[0] + red[1]) + (red[2] + red[3])) / (float)d + eps);
#pragma unroll
    for (int j = 0; j < NV; ++j) {
        const size_t o = base + (j * 256 + t) * 4;
        const float4v y = float4v{v[j][0] * inv * g[j][0], v[j][1] * inv * g[j][1], v[j][2] * inv * g[j][2],
                                  v[j][3] * inv * g[j][3]};
        if constexpr (OM == 1) {
            vsl_half h0, h1, h2, h3, l0, l1, l2, l3;
            split_f16(y[0], h0, l0);
            split_f16(y[1], h1, l1);
            split_f16(y[2], h2, l2);
            split_f16(y[3], h3, l3);
            *reinterpret_cast<half4*>(out + o) = half4{h0, h1, h2, h3};
            *reinterpret_cast<half4*>(out + MN + o) = half4{l0, l1, l2, l3};
        } else if constexpr (OM == 2) {
            half4 h;
            uint32_t lo8;
            split4_f16_f8(y[0], y[1], y[2], y[3], h, lo8);
            *reinterpret_cast<half4*>(out + o) = h;
            *reinterpret_cast<uint32_t*>(reinterpret_cast<uint8_t*>(out + MN) + base + lo8_pos((j * 256 + t) * 4)) = lo8;
        } else if constexpr (sizeof(OT) == 2) {
            *reinterpret_cast<half4*>(out + o) = half4{(vsl_half)y[0], (vsl_half)y[1], (vsl_half)y[2], (vsl_half)y[3]};
        } else {
            *reinterpret_cast<float4v*>(out + o) = y;
        }
    }
}

// ---------------------------------------------------------------------------------------------
// causal flash attention (prefill), fp16 in / fp16 out, fp32 softmax statistics
// ---------------------------------------------------------------------------------------------
// Causal flash attention for one chunk of S prompt rows at positions pos0.. (their K/V already in
// the cache). Block = the G query heads of one KV head x 32 query rows, one wave per head (two for
// G <= 4, each taking one 32-key half of every tile, merged at the end): each
// 64-position K/V tile is copied once for all G heads straight from the cache into LDS
// (global_load_lds, three tile buffers, each tile requested two tiles ahead), both row-major with the
// chunk swizzle of ksw. Per tile each wave computes S^T = K Q^T (two 32-position fragments), the
// online softmax of its 32 query rows (each lane owns one row's statistics with its partner lane
// l^32), and O^T += V^T P^T, whose V^T operand comes from the row-major V tile through LDS
// transpose reads. The next tile's S^T is issued on the matrix cores while the current tile's
// probabilities are computed on the VALU.
constexpr int kAttnTile = 64;  // KV positions per tile

template <int HD>
__device__ __forceinline__ int ksw(int r, int c) {
    if constexpr (HD == 128) return r * HD + ((c ^ (r & 15)) * 8);       // 256-byte rows: 16 rows per bank sweep
    else return r * HD + ((c ^ ((r >> 1) & 7)) * 8);                      // 128-byte rows: row pairs
}

// KSPLIT = 2 / 4: two / four waves per query head, each taking one 32-key block of every tile (its
// own online softmax state), merged through LDS at the end. GB: query heads per block (a divisor of
// G); blockIdx.y = KV head * (G / GB) + the block's group of GB heads. TK keys per tile, NBUF tile
// buffers (3: the next tile's scores are issued while the current tile's probabilities are formed;
// 2: one tile copied ahead, each tile's scores after its copy landed).
template <int HD, int G, int GB, bool QX2, int OM, bool WIN, int KSPLIT, int TK = kAttnTile, int NBUF = 3>
__global__ __launch_bounds__(64 * GB * KSPLIT) void k_attn_prefill(const vsl_half* __restrict__ q, const vsl_half* __restrict__ kc,
                                                         const vsl_half* __restrict__ vc, uint32_t S, uint32_t pos0,
                                                         uint32_t n_q, uint32_t n_kv, uint32_t cap, float scale,
                                                         vsl_half* __restrict__ out, uint32_t win, uint32_t n_glob,
                                                         uint32_t thr) {
    constexpr int NT = 64 * GB * KSPLIT;
    static_assert(G % GB == 0, "heads per block divide the group");
    static_assert(NBUF == 2 || NBUF == 3, "two or three tile buffers");
    constexpr int NKB = TK / 32 / KSPLIT;       // 32-key blocks of a tile per wave
    static_assert(NKB >= 1 && NKB * KSPLIT * 32 == TK, "a tile's key blocks divide over the waves of a head");
    constexpr int CPR = HD / 8;                 // 16-byte chunks per K/V row
    constexpr int NCH = TK * CPR / NT;          // chunks per thread per tile (K and V each)
    constexpr int QP = QX2 ? 2 : 1;             // q planes; with split q the probabilities are split too
    static_assert(NCH >= 1 && TK * CPR % NT == 0, "tile does not divide over the block");
    __shared__ __attribute__((aligned(16))) vsl_half Ks[NBUF][TK * HD];
    __shared__ __attribute__((aligned(16))) vsl_half Vs[NBUF][TK * HD];
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t n_qb = gridDim.x;
    const uint32_t qb = n_qb - 1 - blockIdx.x;  // the longest (latest) query blocks start first
    const uint32_t kvh = blockIdx.y / (G / GB);
    const int ksp = wave / GB;                  // this wave's share of every tile (0 .. KSPLIT-1)
    const int kbase = ksp * NKB;                // its first 32-key block
    const uint32_t h = kvh * G + (blockIdx.y % (G / GB)) * GB + wave % GB;  // kv_head = head * n_kv / n_q
    const uint32_t s_base = qb * 32;
    const uint32_t my_s = s_base + (lane & 31);  // query row owned by this lane (stats, O^T column)
    const uint32_t qw = n_q * HD;
    const size_t qplane = (size_t)S * qw;
    const float sl2 = scale * 1.4426950408889634f;
    const uint32_t last_s = min(S, s_base + 32) - 1;
    const uint32_t kv_end = pos0 + last_s + 1;  // positions 0..kv_end-1 are visible to some row
    const uint32_t my_pos = pos0 + my_s;
    const uint32_t n_tiles = (kv_end + TK - 1) / TK;
    // Windowed rows (position p with p + 1 > thr) see the keys k < n_glob and k >= p - win only.
    // When the block's first row is windowed, every row is, and the key tiles below the first row's
    // window and past the global tiles are skipped: virtual tile vt runs over [0, n_gt) and then
    // [t_lo, n_tiles).
    const uint32_t p_first = pos0 + s_base;
    uint32_t n_gt = n_tiles, t_lo = n_tiles;
    if (WIN && p_first + 1 > thr && p_first > win) {
        t_lo = (p_first - win) / TK;
        n_gt = min((n_glob + TK - 1) / TK, t_lo);
    }
    const uint32_t n_vt = n_gt + (n_tiles - t_lo);
    auto phys = [&](uint32_t vt) { return vt < n_gt ? vt : vt - n_gt + t_lo; };
    // this lane's row: keys below my_lo (and not global) are masked
    const uint32_t my_lo = (WIN && my_pos + 1 > thr && my_pos > win) ? my_pos - win : 0;
    // the largest window start of the block's rows (the last row's: starts grow with the position)
    const uint32_t p_last = pos0 + last_s;
    const uint32_t lo_max = (WIN && p_last + 1 > thr && p_last > win) ? p_last - win : 0;
    const vsl_half* Kb = kc + (size_t)kvh * cap * HD;
    const vsl_half* Vb = vc + (size_t)kvh * cap * HD;

    // Tile copy: LDS chunk position P = i * NT + tid holds row P / CPR and the logical chunk whose
    // swizzled position is P % CPR (the swizzle is an xor, its own inverse). Positions past kv_end
    // copy position 0 (in bounds; finite values whose probabilities are 0).
    uint32_t roff[NCH];  // byte offset of the chunk within a tile, without the tile's first row
    int rrow[NCH];
#pragma unroll
    for (int i = 0; i < NCH; ++i) {
        const int P = i * NT + tid, r = P / CPR;
        const int c = (ksw<HD>(r, P % CPR) - r * HD) / 8;
        rrow[i] = r;
        roff[i] = (uint32_t)(c * 8 * 2);
    }
    auto issue = [&](int buf, uint32_t t) {
#pragma unroll
        for (int i = 0; i < NCH; ++i) {
            const uint32_t pos = t * TK + rrow[i];
            const uint32_t off = (pos < kv_end ? pos : 0u) * (HD * 2) + roff[i];
            lds_load16(Kb, off, &Ks[buf][(i * NT + wave * 64) * 8]);
            lds_load16(Vb, off, &Vs[buf][(i * NT + wave * 64) * 8]);
        }
    };

    // Q^T as the B operand of S^T = K Q^T: lane holds q row (l%32), dims 16c + 8*(l/32)..+7
    half8 qf[QP][HD / 16];
#pragma unroll
    for (int p = 0; p < QP; ++p)
#pragma unroll
        for (int c = 0; c < HD / 16; ++c) {
            const uint32_t row = my_s < S ? my_s : S - 1;  // rows past S are never stored
            qf[p][c] = *reinterpret_cast<const half8*>(q + p * qplane + (size_t)row * qw + (size_t)h * HD + c * 16 +
                                                       (lane >> 5) * 8);
        }
    float16v o[HD / 32];
#pragma unroll
    for (int t = 0; t < HD / 32; ++t)
#pragma unroll
        for (int v = 0; v < 16; ++v) o[t][v] = 0.f;
    float m = -INFINITY, l = 0.f;

    // Lazy rescaling: m is the reference maximum of this lane's row (probabilities are taken as
    // 2^(score - m)); it is raised, and the accumulators rescaled, only when a tile's maximum exceeds
    // it by more than kLazy (log2 units) in some lane of the wave, so every probability stays below
    // 2^kLazy and most tiles skip the rescale. The quotient O / l does not depend on m.
    constexpr float kLazy = 8.f;
    // S^T[kv][q] = sum_d K[kv][d] Q[q][d] for the two 32-position halves of the tile in `buf`
    auto qk = [&](int buf, float16v (&st)[NKB]) {
#pragma unroll
        for (int kb = 0; kb < NKB; ++kb) {
#pragma unroll
            for (int v = 0; v < 16; ++v) st[kb][v] = 0.f;
            half8 kf[HD / 16];
#pragma unroll
            for (int c = 0; c < HD / 16; ++c)
                kf[c] = *reinterpret_cast<const half8*>(
                    &Ks[buf][ksw<HD>((kbase + kb) * 32 + (lane & 31), 2 * c + (lane >> 5))]);
#pragma unroll
            for (int c = 0; c < HD / 16; ++c)
#pragma unroll
                for (int p = 0; p < QP; ++p) st[kb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(kf[c], qf[p][c], st[kb], 0, 0, 0);
        }
    };
    // scaled scores of tile t with the causal (and window) mask, applied only on tiles that reach past
    // the block's first row; returns the tile maximum of this lane's row
    auto mask_max = [&](float16v (&st)[NKB], uint32_t t) {
        float bm = -INFINITY;
        // wave-uniform: every key of the tile is visible to every row of the block (at or below the
        // first row, and inside every row's window or among the global keys)
        if (t * TK + TK - 1 <= p_first && (!WIN || t * TK >= lo_max || t * TK + TK - 1 < n_glob)) {
#pragma unroll
            for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
                for (int v = 0; v < 16; ++v) {
                    st[kb][v] *= sl2;
                    bm = fmaxf(bm, st[kb][v]);
                }
        } else {
#pragma unroll
            for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
                for (int v = 0; v < 16; ++v) {
                    const uint32_t kvp = t * TK + (kbase + kb) * 32 + d_row(v, lane);
                    const bool seen = WIN ? kvp <= my_pos && (kvp >= my_lo || kvp < n_glob) : kvp <= my_pos;
                    st[kb][v] = seen ? st[kb][v] * sl2 : -INFINITY;
                    bm = fmaxf(bm, st[kb][v]);
                }
        }
        float ba, bb;
        lane_pair<32>(bm, ba, bb);
        return fmaxf(ba, bb);
    };
    auto rescale = [&](float bm) {
        const bool raise = bm > m + kLazy;  // m = -inf: any finite tile maximum raises it
        if (__builtin_amdgcn_ballot_w64(raise)) {
            const float mn = raise ? bm : m;
            const float corr = mn == -INFINITY ? 1.f : fast_exp2(m - mn);  // m = -inf: 0
            l *= corr;
            m = mn;
#pragma unroll
            for (int tt = 0; tt < HD / 32; ++tt)
#pragma unroll
                for (int v = 0; v < 16; ++v) o[tt][v] *= corr;
        }
    };
    // probabilities 2^(score - m) as the P^T operand (split into hi / lo planes with a split q);
    // returns their sum over the tile for this lane's row
    auto probs = [&](const float16v (&st)[NKB], half8 (&pf)[QP][NKB][2]) {
        float ps = 0.f;
#pragma unroll
        for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
            for (int v = 0; v < 16; ++v) {
                const float pv = (st[kb][v] == -INFINITY) ? 0.f : fast_exp2(st[kb][v] - m);
                ps += pv;
                if constexpr (QX2) {
                    vsl_half hi, lo;
                    split_f16(pv, hi, lo);
                    pf[0][kb][v >> 3][v & 7] = hi;
                    pf[QP - 1][kb][v >> 3][v & 7] = lo;
                } else {
                    pf[0][kb][v >> 3][v & 7] = (vsl_half)pv;
                }
            }
        float pa, pb;
        lane_pair<32>(ps, pa, pb);
        return pa + pb;
    };
    // O^T[dim][q] += sum_kv V^T[dim][kv] P^T[kv][q]; P^T slots v = 0..7 / 8..15 of each half are
    // the kv rows (v/4)*8 + (l/32)*4 + v%4, which the V^T operand reads to match: lane l needs
    // V[r0 + j][dim] and V[r0 + 8 + j][dim] (j = 0..3) for dim = 32 tt + l%32, r0 = 32 kb + 16 hi
    // + 4 (l/32). ds_read_b64_tr_b16 gives lane i of a 16-lane group element i%4 of the 8-byte
    // row addressed by lane 4j + i/4 of the group as its value j, so lane i addresses
    // V[r0 + i/4][d0 + 4 (i%4) .. +3] with d0 the group's first dim: value j is V[r0 + j][d0 + i].
    auto pv = [&](int buf, const half8 (&pf)[QP][NKB][2]) {
        const vsl_half* Vt = Vs[buf];
        const int gi = lane & 15, gdim = ((lane >> 4) & 1) * 16 + 4 * (gi & 3);
#pragma unroll
        for (int tt = 0; tt < HD / 32; ++tt) {
            const int d = tt * 32 + gdim;
#pragma unroll
            for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
                for (int hi = 0; hi < 2; ++hi) {
                    const int r = (kbase + kb) * 32 + hi * 16 + (lane >> 5) * 4 + (gi >> 2);
                    const half4 x0 = lds_read_tr16(Vt + ksw<HD>(r, d >> 3) + (d & 7));
                    const half4 x1 = lds_read_tr16(Vt + ksw<HD>(r + 8, d >> 3) + (d & 7));
                    const half8 af = half8{x0[0], x0[1], x0[2], x0[3], x1[0], x1[1], x1[2], x1[3]};
#pragma unroll
                    for (int p = 0; p < QP; ++p)
                        o[tt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af, pf[p][kb][hi], o[tt], 0, 0, 0);
                }
        }
    };

    // Tile pipeline over three buffers. At the top of iteration t tiles t and t+1 are in LDS and the
    // scores of tile t are in registers: tile t+2 is requested into the buffer tile t-1 used, tile
    // t's scores are masked and its maximum taken (the lazy rescale is the one branch), then tile
    // t+1's scores are issued on the matrix cores while the VALU turns tile t's scores into
    // probabilities (independent work in one basic block, so the two overlap), then tile t's PV
    // products; each wave waits for its own copies and the block meets at a barrier (every copy of
    // t+2 is in LDS, every wave has finished reading buffer t, which iteration t+1 overwrites).
    // Requests past the last tile re-copy it (finite values; scores computed from them are unused).
    if constexpr (NBUF == 3) {
        auto buf_of = [](uint32_t t) { return (int)(t % 3); };
        issue(0, phys(0));
        issue(1, phys(n_vt > 1 ? 1 : 0));
        VSL_VMCNT_WAIT(0);
        __syncthreads();
        float16v st[NKB];
        qk(0, st);
        for (uint32_t t = 0; t < n_vt; ++t) {
            issue(buf_of(t + 2), phys(t + 2 < n_vt ? t + 2 : n_vt - 1));
            rescale(mask_max(st, phys(t)));
            float16v sn[NKB];
            qk(buf_of(t + 1), sn);
            half8 pf[QP][NKB][2];
            l += probs(st, pf);
            pv(buf_of(t), pf);
#pragma unroll
            for (int kb = 0; kb < NKB; ++kb) st[kb] = sn[kb];
            VSL_VMCNT_WAIT(0);
            __syncthreads();
        }
    } else {
        // two buffers: tile t+1 is copied into the buffer tile t-1 used (free since the barrier that
        // ended iteration t-1) while tile t is computed; each wave waits for its own copies and the
        // block meets at a barrier before tile t+1 is read
        issue(0, phys(0));
        VSL_VMCNT_WAIT(0);
        __syncthreads();
        for (uint32_t t = 0; t < n_vt; ++t) {
            issue((int)((t + 1) & 1), phys(t + 1 < n_vt ? t + 1 : n_vt - 1));
            float16v st[NKB];
            qk((int)(t & 1), st);
            rescale(mask_max(st, phys(t)));
            half8 pf[QP][NKB][2];
            l += probs(st, pf);
            pv((int)(t & 1), pf);
            VSL_VMCNT_WAIT(0);
            __syncthreads();
        }
    }

    if constexpr (KSPLIT > 1) {
        // merge the key shares of each head: waves with ksp > 0 leave their accumulators and row
        // statistics in the (now unused) tile buffers, the ksp = 0 wave rescales all to the largest
        // maximum (every buffer read and every copy landed at the loop's last barrier)
        constexpr int OSZ = HD / 32 * 16 * 64;  // accumulator floats per wave
        constexpr int SLOT = OSZ + 128;
        const int hw = wave % GB;
        static_assert(KSPLIT == 2 ? 2 * SLOT * 4 <= NBUF * TK * HD * 2 : (KSPLIT - 1) * SLOT * 4 <= NBUF * TK * HD * 2,
                      "merge area exceeds a tile buffer set");
        static_assert(KSPLIT == 2 || GB <= 2, "four shares per head: at most two heads per block");
        // slot of (head hw, share j >= 1): KSPLIT = 2 packs two heads per buffer set, KSPLIT = 4 gives
        // each head its own set (K buffers for head 0, V buffers for head 1)
        auto slot = [&](int j) {
            if constexpr (KSPLIT == 2) return reinterpret_cast<float*>(hw < 2 ? &Ks[0][0] : &Vs[0][0]) + (hw & 1) * SLOT;
            else return reinterpret_cast<float*>(hw == 0 ? &Ks[0][0] : &Vs[0][0]) + (j - 1) * SLOT;
        };
        if (ksp > 0) {
            float* xo = slot(ksp);
#pragma unroll
            for (int tt = 0; tt < HD / 32; ++tt)
#pragma unroll
                for (int v = 0; v < 16; ++v) xo[(tt * 16 + v) * 64 + lane] = o[tt][v];
            xo[OSZ + lane] = m;
            xo[OSZ + 64 + lane] = l;
        }
        __syncthreads();
        if (ksp > 0) return;
        float mm = m;
#pragma unroll
        for (int j = 1; j < KSPLIT; ++j) mm = fmaxf(mm, slot(j)[OSZ + lane]);
        const float c0 = m == -INFINITY ? 0.f : fast_exp2(m - mm);
        l *= c0;
#pragma unroll
        for (int tt = 0; tt < HD / 32; ++tt)
#pragma unroll
            for (int v = 0; v < 16; ++v) o[tt][v] *= c0;
#pragma unroll
        for (int j = 1; j < KSPLIT; ++j) {
            const float* xo = slot(j);
            const float mj = xo[OSZ + lane];
            const float cj = mj == -INFINITY ? 0.f : fast_exp2(mj - mm);
            l += xo[OSZ + 64 + lane] * cj;
#pragma unroll
            for (int tt = 0; tt < HD / 32; ++tt)
#pragma unroll
                for (int v = 0; v < 16; ++v) o[tt][v] += xo[(tt * 16 + v) * 64 + lane] * cj;
        }
    }

    if (my_s >= S) return;
    const float inv = l > 0.f ? 1.f / l : 0.f;
    vsl_half* orow = out + (size_t)my_s * qw + (size_t)h * HD;
    // element v of O^T fragment t is dim 32 t + d_row(v, lane): runs of 4 consecutive dims (v%4), so
    // each run is one 8-byte store per plane
#pragma unroll
    for (int t = 0; t < HD / 32; ++t)
#pragma unroll
        for (int v0 = 0; v0 < 16; v0 += 4) {
            half4 hv, lv;
            const int dim = t * 32 + d_row(v0, lane);
            if constexpr (OM == 2) {
                uint32_t lo8;
                split4_f16_f8(o[t][v0] * inv, o[t][v0 + 1] * inv, o[t][v0 + 2] * inv, o[t][v0 + 3] * inv, hv, lo8);
                *reinterpret_cast<half4*>(orow + dim) = hv;
                // the lo8 plane (bytes) follows the hi plane; columns h HD + dim .. + 3 stay contiguous
                *reinterpret_cast<uint32_t*>(reinterpret_cast<uint8_t*>(out + qplane) + (size_t)my_s * qw +
                                             lo8_pos(h * HD + dim)) = lo8;
                continue;
            }
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float val = o[t][v0 + i] * inv;
                if constexpr (OM == 1) {
                    vsl_half hi, lo;
                    split_f16(val, hi, lo);
                    hv[i] = hi;
                    lv[i] = lo;
                } else {
                    hv[i] = (vsl_half)val;
                }
            }
            *reinterpret_cast<half4*>(orow + dim) = hv;
            if constexpr (OM == 1) *reinterpret_cast<half4*>(orow + qplane + dim) = lv;
        }
}

}  // namespace

template <class G, int EPI>
static void launch_gemm_cfg(uint32_t blocks, hipStream_t s, const vsl_half* a, const vsl_half* b, uint32_t M,
                            uint32_t N, uint32_t K, void* C, bool ax2, bool cx2) {
    if (ax2 && cx2) k_gemm_f16<G, EPI, true, true><<<blocks, G::NT, 0, s>>>(a, b, M, N, K, C);
    else if (ax2) k_gemm_f16<G, EPI, true, false><<<blocks, G::NT, 0, s>>>(a, b, M, N, K, C);
    else if (cx2) k_gemm_f16<G, EPI, false, true><<<blocks, G::NT, 0, s>>>(a, b, M, N, K, C);
    else k_gemm_f16<G, EPI, false, false><<<blocks, G::NT, 0, s>>>(a, b, M, N, K, C);
}

template <class G, int EPI>
static uint32_t gemm_tiles(uint32_t M, uint32_t N) {
    const uint32_t ncols = EPI == VSL_EPI_SWIGLU ? G::BN / 2 : G::BN;
    return N % ncols ? 0u : ((M + G::BM - 1) / G::BM) * (N / ncols);
}

constexpr uint32_t kDmaMinTiles = 192;

// A operand form of a GEMM's flags (the caller has rejected A_X2 | A_F8 together)
static int gemm_a_mode(int flags) {
    return (flags & VSL_GEMM_A_X2) ? kGemmAX2 : (flags & VSL_GEMM_A_F8) ? kGemmAF8 : kGemmA1;
}

constexpr int kB8Field = 0xFF << 16;  // the VSL_GEMM_B8_SHIFT field of the flags

// The weight shift of a GEMM's flags (VSL_GEMM_B8_SHIFT_DEFAULT without the field); false when the
// field is outside [VSL_GEMM_B8_SHIFT_MIN, VSL_GEMM_B8_SHIFT_MAX].
static bool gemm_b8_shift(int flags, int* shift) {
    const int f = (flags & kB8Field) >> 16;
    *shift = f ? f - 128 : VSL_GEMM_B8_SHIFT_DEFAULT;
    return *shift >= VSL_GEMM_B8_SHIFT_MIN && *shift <= VSL_GEMM_B8_SHIFT_MAX;
}

// The A-operand flags of the stage entries: A_X2 or A_F8 (not both), a weight shift in range.
static bool a_flags_valid(int a_flags, int* shift) {
    const int form = a_flags & (VSL_GEMM_A_X2 | VSL_GEMM_A_F8);
    return !(a_flags & ~(VSL_GEMM_A_X2 | VSL_GEMM_A_F8 | kB8Field)) && form != (VSL_GEMM_A_X2 | VSL_GEMM_A_F8) &&
           gemm_b8_shift(a_flags, shift);
}

// The K split launch_gemm takes for a shape and workspace (0: unsplit kernels).
static uint32_t splitk_choice(uint32_t M, uint32_t N, uint32_t K, int epi, const float* ws, uint64_t ws_bytes) {
    for (int cfg = 0; cfg < 2; ++cfg)
        if (vsl_gemm_dma_tiles(cfg, M, N, K, epi) >= kDmaMinTiles) return 0;
    if (!ws) return 0;
    uint64_t need = 0;
    const uint32_t ks = vsl_gemm_splitk_plan(M, N, K, epi, kDmaMinTiles, &need);
    return ks && need <= ws_bytes ? ks : 0;
}

static bool aligned_to(const void* p, uintptr_t a) { return (reinterpret_cast<uintptr_t>(p) & (a - 1)) == 0; }

// Tile configuration by occupancy: the largest tiles that still give every CU a tile.
template <int EPI>
static int launch_gemm(hipStream_t s, const vsl_half* a, const vsl_half* b, uint32_t M, uint32_t N, uint32_t K,
                       void* C, int am, int cm, float* ws, uint64_t ws_bytes, int b8s) {
    auto blocks = [](uint32_t tiles) { return ((tiles + 7) / 8) * 8; };  // whole XCD ranges (tile_of)
    // shapes whose 256 x 256 (else 128 x 256) tiles cover at least three quarters of the CUs take
    // the direct-to-LDS kernel
    for (int cfg = 0; cfg < 2; ++cfg)
        if (vsl_gemm_dma_tiles(cfg, M, N, K, EPI) >= kDmaMinTiles)
            return vsl_gemm_dma_launch(cfg, s, a, b, M, N, K, C, EPI, am, cm, b8s) == 0
                       ? VSL_OK
                       : vsl_invalid("vsl_gemm_f16: shape %ux%ux%u does not fit the direct-to-LDS tiles", M, N, K);
    // otherwise, with a workspace, split K over enough blocks
    if (const uint32_t ks = splitk_choice(M, N, K, EPI, ws, ws_bytes)) {
        if (vsl_gemm_splitk_launch(ks, s, a, b, M, N, K, C, EPI, am, ws, b8s))
            return vsl_invalid("vsl_gemm_f16: split-K epilogue %d", EPI);
        return VSL_OK;
    }
    // the fp8 lo forms exist in the direct-to-LDS kernel only: on shapes its 128 x 256 tiles take, its
    // 64 x 128 tiles where those cover the CUs (no workspace: O of a 512-row chunk 94 -> 56 us with its
    // RMSNorm), else its larger tiles even when they leave CUs idle
    if (am == kGemmAF8 || cm == kGemmCF8) {
        if (vsl_gemm_dma_tiles(1, M, N, K, EPI) && vsl_gemm_dma_tiles(2, M, N, K, EPI) >= kDmaMinTiles &&
            vsl_gemm_dma_launch(2, s, a, b, M, N, K, C, EPI, am, cm, b8s) == 0)
            return VSL_OK;
        for (int cfg = 1; cfg >= 0; --cfg)
            if (vsl_gemm_dma_tiles(cfg, M, N, K, EPI) &&
                vsl_gemm_dma_launch(cfg, s, a, b, M, N, K, C, EPI, am, cm, b8s) == 0)
                return VSL_OK;
        return vsl_unsupported("vsl_gemm_f16: F16F8 operands need N %% 256 == 0 (128 for SwiGLU) and K %% 128 == 0 "
                               "(shape %ux%ux%u)", M, N, K);
    }
    // few rows without a K split (e.g. a 128-row prompt's SwiGLU): the 64 x 128 direct-to-LDS tiles
    if (vsl_gemm_dma_tiles(2, M, N, K, EPI) >= kDmaMinTiles &&
        vsl_gemm_dma_launch(2, s, a, b, M, N, K, C, EPI, am, cm, b8s) == 0)
        return VSL_OK;
    const bool ax2 = am == kGemmAX2, cx2 = cm == kGemmCX2;
    const uint32_t tb = gemm_tiles<GemmBig, EPI>(M, N), tm = gemm_tiles<GemmMid, EPI>(M, N);
    const uint32_t ts = gemm_tiles<GemmSmall, EPI>(M, N);
    if (tb >= 256) launch_gemm_cfg<GemmBig, EPI>(blocks(tb), s, a, b, M, N, K, C, ax2, cx2);
    else if (tm >= 256) launch_gemm_cfg<GemmMid, EPI>(blocks(tm), s, a, b, M, N, K, C, ax2, cx2);
    else if (ts) launch_gemm_cfg<GemmSmall, EPI>(blocks(ts), s, a, b, M, N, K, C, ax2, cx2);
    else return vsl_invalid("vsl_gemm_f16: N=%u is not a multiple of the tile width", N);
    return VSL_OK;
}

static int gemm_f16(const void* A, const void* B, uint32_t M, uint32_t N, uint32_t K, void* C, int epilogue,
                    float* ws, uint64_t ws_bytes, void* stream) {
    if (!A || !B || !C) return vsl_invalid("vsl_gemm_f16: null pointer");
    if (M == 0) return VSL_OK;
    const int epi = epilogue & 0xFF;
    int b8s = 0;
    if ((epilogue & ~(0xFF | VSL_GEMM_A_X2 | VSL_GEMM_C_X2 | VSL_GEMM_A_F8 | VSL_GEMM_C_F8 | kB8Field)) ||
        (epilogue & (VSL_GEMM_A_X2 | VSL_GEMM_A_F8)) == (VSL_GEMM_A_X2 | VSL_GEMM_A_F8) ||
        (epilogue & (VSL_GEMM_C_X2 | VSL_GEMM_C_F8)) == (VSL_GEMM_C_X2 | VSL_GEMM_C_F8) || !gemm_b8_shift(epilogue, &b8s))
        return vsl_invalid("vsl_gemm_f16: flags 0x%x", epilogue);
    const int am = gemm_a_mode(epilogue);
    const int cm = (epilogue & VSL_GEMM_C_X2) ? kGemmCX2 : (epilogue & VSL_GEMM_C_F8) ? kGemmCF8 : kGemmC1;
    if (cm != kGemmC1 && epi != VSL_EPI_SWIGLU) return vsl_invalid("vsl_gemm_f16: C_X2 / C_F8 need VSL_EPI_SWIGLU");
    if (K % 32) return vsl_invalid("vsl_gemm_f16: K=%u must be a multiple of 32", K);
    const uint32_t ncols = epi == VSL_EPI_SWIGLU ? 64 : 128;
    if (N % ncols) return vsl_invalid("vsl_gemm_f16: N=%u must be a multiple of %u", N, ncols);
    hipStream_t s = static_cast<hipStream_t>(stream);
    const vsl_half* a = static_cast<const vsl_half*>(A);
    const vsl_half* b = static_cast<const vsl_half*>(B);
    int rc;
    switch (epi) {
        case VSL_EPI_STORE_F32: rc = launch_gemm<VSL_EPI_STORE_F32>(s, a, b, M, N, K, C, am, kGemmC1, ws, ws_bytes, b8s); break;
        case VSL_EPI_STORE_F16: rc = launch_gemm<VSL_EPI_STORE_F16>(s, a, b, M, N, K, C, am, kGemmC1, ws, ws_bytes, b8s); break;
        case VSL_EPI_RESID: rc = launch_gemm<VSL_EPI_RESID>(s, a, b, M, N, K, C, am, kGemmC1, ws, ws_bytes, b8s); break;
        case VSL_EPI_SWIGLU: rc = launch_gemm<VSL_EPI_SWIGLU>(s, a, b, M, N, K, C, am, cm, ws, ws_bytes, b8s); break;
        default: return vsl_invalid("vsl_gemm_f16: epilogue %d", epi);
    }
    if (rc) return rc;
    HIP_TRY(hipGetLastError());
    return VSL_OK;
}

extern "C" int vsl_gemm_f16(const void* A, const void* B, uint32_t M, uint32_t N, uint32_t K, void* C, int epilogue,
                            void* stream) {
    return gemm_f16(A, B, M, N, K, C, epilogue, nullptr, 0, stream);
}

extern "C" int vsl_gemm_f16_ws(const void* A, const void* B, uint32_t M, uint32_t N, uint32_t K, void* C,
                               int epilogue, void* workspace, uint64_t ws_bytes, void* stream) {
    if (workspace && (reinterpret_cast<uintptr_t>(workspace) & 15))
        return vsl_invalid("vsl_gemm_f16_ws: workspace must be 16-byte aligned");
    return gemm_f16(A, B, M, N, K, C, epilogue, static_cast<float*>(workspace), workspace ? ws_bytes : 0, stream);
}

extern "C" int vsl_gemm_f16_direct(uint32_t M, uint32_t N, uint32_t K, int epilogue) {
    const int epi = epilogue & 0xFF;
    for (int cfg = 0; cfg < 2; ++cfg)
        if (vsl_gemm_dma_tiles(cfg, M, N, K, epi) >= kDmaMinTiles) return 1;
    return vsl_gemm_splitk_plan(M, N, K, epi, kDmaMinTiles, nullptr) ? 1 : 0;
}

extern "C" uint64_t vsl_gemm_f16_ws_bytes(uint32_t M, uint32_t N, uint32_t K, int epilogue) {
    const int epi = epilogue & 0xFF;
    for (int cfg = 0; cfg < 2; ++cfg)
        if (vsl_gemm_dma_tiles(cfg, M, N, K, epi) >= kDmaMinTiles) return 0;
    uint64_t need = 0;
    return vsl_gemm_splitk_plan(M, N, K, epi, kDmaMinTiles, &need) ? need : 0;
}

// RoPE + Q/K/V split of KS partials (KS = 1: the finished projection), four columns per thread.
template <int KS>
static void launch_rope_split4(hipStream_t s, const float* ws, uint32_t S, uint32_t n_q, uint32_t n_kv, uint32_t hd,
                               uint32_t pos0, const float* rc, const float* rsn, vsl_half* qo, bool qx2, void* kc,
                               void* vc, bool kv32, uint32_t cap, uint32_t ks_rt = KS) {
    const uint64_t quads = (uint64_t)S * (n_q + 2 * n_kv) * hd / 4;
    const uint32_t grid = (uint32_t)((quads + 255) / 256);
    if (!kv32) {
        if (qx2) k_rope_split4<WF16, true, KS><<<grid, 256, 0, s>>>(ws, S, n_q, n_kv, hd, pos0, rc, rsn, qo, kc, vc, cap, ks_rt);
        else k_rope_split4<WF16, false, KS><<<grid, 256, 0, s>>>(ws, S, n_q, n_kv, hd, pos0, rc, rsn, qo, kc, vc, cap, ks_rt);
    } else {
        if (qx2) k_rope_split4<WF32, true, KS><<<grid, 256, 0, s>>>(ws, S, n_q, n_kv, hd, pos0, rc, rsn, qo, kc, vc, cap, ks_rt);
        else k_rope_split4<WF32, false, KS><<<grid, 256, 0, s>>>(ws, S, n_q, n_kv, hd, pos0, rc, rsn, qo, kc, vc, cap, ks_rt);
    }
}

// Arguments of the RoPE + split step; VSL_OK or the error code (nothing launched on error).
static int check_rope_split(const char* fn, const void* qkv, uint32_t S, uint32_t hd, uint32_t pos0,
                            const float* rope_cos, const float* rope_sin, const void* q_out, int q_dtype,
                            const void* kcache, const void* vcache, int kv_dtype, uint32_t cap) {
    if (!qkv || !rope_cos || !rope_sin || !q_out || !kcache || !vcache) return vsl_invalid("%s: null pointer", fn);
    if ((uint64_t)pos0 + S > cap) {
        vsl_set_error("%s: positions %u..%u exceed capacity %u", fn, pos0, pos0 + S - 1, cap);
        return VSL_E_CAPACITY;
    }
    if (hd % 2) return vsl_invalid("%s: odd head_dim", fn);
    if (q_dtype != VSL_DT_F16 && q_dtype != VSL_DT_F16X2) return vsl_unsupported("%s: q dtype %d", fn, q_dtype);
    if (kv_dtype != VSL_DT_F16 && kv_dtype != VSL_DT_F32) return vsl_unsupported("%s: kv dtype %d", fn, kv_dtype);
    return VSL_OK;
}

// The four-column kernel's layout needs: hd % 4, 16-byte partials, 8-byte tables and q, caches
// aligned to four elements.
static bool rope_split4_fits(const void* ws, uint32_t hd, const float* rc, const float* rsn, const void* q,
                             const void* kc, const void* vc, bool kv32) {
    const uintptr_t ca = kv32 ? 16 : 8;
    return hd % 4 == 0 && aligned_to(ws, 16) && aligned_to(rc, 8) && aligned_to(rsn, 8) && aligned_to(q, 8) &&
           aligned_to(kc, ca) && aligned_to(vc, ca);
}

extern "C" int vsl_rope_split_append(const float* qkv, uint32_t S, uint32_t n_q, uint32_t n_kv, uint32_t hd, uint32_t pos0,
                                     const float* rope_cos, const float* rope_sin, void* q_out, int q_dtype,
                                     void* kcache, void* vcache, int kv_dtype, uint32_t cap, void* stream) {
    if (const int rc = check_rope_split("vsl_rope_split_append", qkv, S, hd, pos0, rope_cos, rope_sin, q_out, q_dtype,
                                        kcache, vcache, kv_dtype, cap))
        return rc;
    if (S == 0) return VSL_OK;
    hipStream_t s = static_cast<hipStream_t>(stream);
    vsl_half* qo = static_cast<vsl_half*>(q_out);
    const bool x2 = q_dtype == VSL_DT_F16X2, kv32 = kv_dtype == VSL_DT_F32;
    if (rope_split4_fits(qkv, hd, rope_cos, rope_sin, q_out, kcache, vcache, kv32)) {
        launch_rope_split4<1>(s, qkv, S, n_q, n_kv, hd, pos0, rope_cos, rope_sin, qo, x2, kcache, vcache, kv32, cap);
        HIP_TRY(hipGetLastError());
        return VSL_OK;
    }
    const uint64_t total = (uint64_t)S * (n_q + 2 * n_kv) * hd / 2;
    const uint32_t grid = (uint32_t)std::min<uint64_t>((total + 255) / 256, 65536);
    if (!kv32) {
        if (x2) k_rope_split<WF16, true><<<grid, 256, 0, s>>>(qkv, S, n_q, n_kv, hd, pos0, rope_cos, rope_sin, qo, kcache, vcache, cap);
        else k_rope_split<WF16, false><<<grid, 256, 0, s>>>(qkv, S, n_q, n_kv, hd, pos0, rope_cos, rope_sin, qo, kcache, vcache, cap);
    } else {
        if (x2) k_rope_split<WF32, true><<<grid, 256, 0, s>>>(qkv, S, n_q, n_kv, hd, pos0, rope_cos, rope_sin, qo, kcache, vcache, cap);
        else k_rope_split<WF32, false><<<grid, 256, 0, s>>>(qkv, S, n_q, n_kv, hd, pos0, rope_cos, rope_sin, qo, kcache, vcache, cap);
    }
    HIP_TRY(hipGetLastError());
    return VSL_OK;
}

extern "C" int vsl_gemm_f16_qkv_rope_append(const void* A, const void* Wqkv, uint32_t S, uint32_t K, int a_flags,
                                            uint32_t n_q, uint32_t n_kv, uint32_t hd, uint32_t pos0,
                                            const float* rope_cos, const float* rope_sin, void* q_out, int q_dtype,
                                            void* kcache, void* vcache, int kv_dtype, uint32_t cap, float* qkv,
                                            void* workspace, uint64_t ws_bytes, void* stream) {
    const char* fn = "vsl_gemm_f16_qkv_rope_append";
    if (!A || !Wqkv) return vsl_invalid("%s: null pointer", fn);
    int b8s = 0;
    if (!a_flags_valid(a_flags, &b8s)) return vsl_invalid("%s: flags 0x%x", fn, a_flags);
    if (const int rc = check_rope_split(fn, qkv, S, hd, pos0, rope_cos, rope_sin, q_out, q_dtype, kcache, vcache,
                                        kv_dtype, cap))
        return rc;
    if (workspace && !aligned_to(workspace, 16)) return vsl_invalid("%s: workspace must be 16-byte aligned", fn);
    if (S == 0) return VSL_OK;
    const uint32_t N = (n_q + 2 * n_kv) * hd;
    float* ws = static_cast<float*>(workspace);
    const bool x2 = q_dtype == VSL_DT_F16X2, kv32 = kv_dtype == VSL_DT_F32;
    const uint32_t ks = splitk_choice(S, N, K, VSL_EPI_STORE_F32, ws, ws ? ws_bytes : 0);
    if (ks && rope_split4_fits(ws, hd, rope_cos, rope_sin, q_out, kcache, vcache, kv32)) {
        hipStream_t s = static_cast<hipStream_t>(stream);
        vsl_half* qo = static_cast<vsl_half*>(q_out);
        vsl_gemm_splitk_partials(ks, stream, A, Wqkv, S, N, K, gemm_a_mode(a_flags), ws, b8s);
        switch (ks) {
            case 2: launch_rope_split4<2>(s, ws, S, n_q, n_kv, hd, pos0, rope_cos, rope_sin, qo, x2, kcache, vcache, kv32, cap); break;
            case 4: launch_rope_split4<4>(s, ws, S, n_q, n_kv, hd, pos0, rope_cos, rope_sin, qo, x2, kcache, vcache, kv32, cap); break;
            case 8: launch_rope_split4<8>(s, ws, S, n_q, n_kv, hd, pos0, rope_cos, rope_sin, qo, x2, kcache, vcache, kv32, cap); break;
            default: launch_rope_split4<0>(s, ws, S, n_q, n_kv, hd, pos0, rope_cos, rope_sin, qo, x2, kcache, vcache, kv32, cap, ks); break;
        }
        HIP_TRY(hipGetLastError());
        return VSL_OK;
    }
    if (const int rc = gemm_f16(A, Wqkv, S, N, K, qkv, VSL_EPI_STORE_F32 | a_flags, ws, ws ? ws_bytes : 0, stream))
        return rc;
    return vsl_rope_split_append(qkv, S, n_q, n_kv, hd, pos0, rope_cos, rope_sin, q_out, q_dtype, kcache, vcache,
                                 kv_dtype, cap, stream);
}

template <typename OT, int X2, int NV>
static void launch_resid_rmsnorm_nv(hipStream_t s, uint32_t ks, const float* ws, uint32_t rows, float* x,
                                    const float* gamma, float eps, OT* out) {
    switch (ks) {
        case 2: k_splitk_resid_rmsnorm<OT, X2, NV, 2><<<rows, 256, 0, s>>>(ws, rows, x, gamma, eps, out, ks); break;
        case 4: k_splitk_resid_rmsnorm<OT, X2, NV, 4><<<rows, 256, 0, s>>>(ws, rows, x, gamma, eps, out, ks); break;
        case 8: k_splitk_resid_rmsnorm<OT, X2, NV, 8><<<rows, 256, 0, s>>>(ws, rows, x, gamma, eps, out, ks); break;
        default: k_splitk_resid_rmsnorm<OT, X2, NV, 0><<<rows, 256, 0, s>>>(ws, rows, x, gamma, eps, out, ks); break;
    }
}

template <typename OT, int X2>
static void launch_resid_rmsnorm(hipStream_t s, uint32_t ks, const float* ws, uint32_t rows, uint32_t d, float* x,
                                 const float* gamma, float eps, OT* out) {
    switch (d / 1024) {
        case 1: launch_resid_rmsnorm_nv<OT, X2, 1>(s, ks, ws, rows, x, gamma, eps, out); break;
        case 2: launch_resid_rmsnorm_nv<OT, X2, 2>(s, ks, ws, rows, x, gamma, eps, out); break;
        case 4: launch_resid_rmsnorm_nv<OT, X2, 4>(s, ks, ws, rows, x, gamma, eps, out); break;
        default: launch_resid_rmsnorm_nv<OT, X2, 8>(s, ks, ws, rows, x, gamma, eps, out); break;
    }
}

extern "C" int vsl_gemm_f16_resid_rmsnorm(const void* A, const void* B, uint32_t M, uint32_t N, uint32_t K,
                                          int a_flags, float* x, const float* gamma, float eps, void* xn,
                                          int xn_dtype, void* workspace, uint64_t ws_bytes, void* stream) {
    const char* fn = "vsl_gemm_f16_resid_rmsnorm";
    if (!A || !B || !x || !xn || N == 0) return vsl_invalid("%s: bad arguments", fn);
    int b8s = 0;
    if (!a_flags_valid(a_flags, &b8s)) return vsl_invalid("%s: flags 0x%x", fn, a_flags);
    if (xn_dtype != VSL_DT_F16 && xn_dtype != VSL_DT_F16X2 && xn_dtype != VSL_DT_F16F8 && xn_dtype != VSL_DT_F32)
        return vsl_unsupported("%s: dtype %d", fn, xn_dtype);
    if (xn_dtype == VSL_DT_F16F8 && N % 32) return vsl_invalid("%s: F16F8 needs N %% 32 == 0 (N = %u)", fn, N);
    if (workspace && !aligned_to(workspace, 16)) return vsl_invalid("%s: workspace must be 16-byte aligned", fn);
    if (M == 0) return VSL_OK;
    float* ws = static_cast<float*>(workspace);
    const uint32_t ks = splitk_choice(M, N, K, VSL_EPI_RESID, ws, ws ? ws_bytes : 0);
    const uint32_t nv = N / 1024;
    // (the unrolled sums hold up to 32 float4 of partials per thread; more than 8 partials take the
    // loop of the runtime-count variant)
    const bool fused = ks && N % 1024 == 0 && (nv == 1 || nv == 2 || nv == 4 || nv == 8) && (ks > 8 || ks * nv <= 32) &&
                       aligned_to(x, 16) && aligned_to(gamma, 16) && aligned_to(xn, xn_dtype == VSL_DT_F32 ? 16 : 8);
    if (!fused) {
        if (const int rc = gemm_f16(A, B, M, N, K, x, VSL_EPI_RESID | a_flags, ws, ws ? ws_bytes : 0, stream)) return rc;
        return vsl_rmsnorm(x, gamma, M, N, eps, xn, xn_dtype, stream);
    }
    hipStream_t s = static_cast<hipStream_t>(stream);
    vsl_gemm_splitk_partials(ks, stream, A, B, M, N, K, gemm_a_mode(a_flags), ws, b8s);
    if (xn_dtype == VSL_DT_F16)
        launch_resid_rmsnorm<vsl_half, 0>(s, ks, ws, M, N, x, gamma, eps, static_cast<vsl_half*>(xn));
    else if (xn_dtype == VSL_DT_F16X2)
        launch_resid_rmsnorm<vsl_half, 1>(s, ks, ws, M, N, x, gamma, eps, static_cast<vsl_half*>(xn));
    else if (xn_dtype == VSL_DT_F16F8)
        launch_resid_rmsnorm<vsl_half, 2>(s, ks, ws, M, N, x, gamma, eps, static_cast<vsl_half*>(xn));
    else
        launch_resid_rmsnorm<float, 0>(s, ks, ws, M, N, x, gamma, eps, static_cast<float*>(xn));
    HIP_TRY(hipGetLastError());
    return VSL_OK;
}

struct PrefillWindow {
    bool on;
    uint32_t win, n_glob, thr;
};

template <int HD, int G, bool WIN>
static void launch_attn_prefill_w(dim3 grid, hipStream_t s, const vsl_half* q, const vsl_half* k, const vsl_half* v,
                                  uint32_t S, uint32_t pos0, uint32_t n_q, uint32_t n_kv, uint32_t cap, float scale,
                                  vsl_half* o, bool qx2, int om, const PrefillWindow& w) {
    // two waves per query head (each half of every key tile) where the merge area -- the tile buffers
    // -- holds the heads' accumulators: 8B shapes, S = 512 / 2048 rows at 0 / 2048 at 6144: 25.9 /
    // 150 / 543 -> 25.1 / 142 / 511 us. Groups of 4 heads are split over two blocks when a block per
    // (32 rows, KV head) would leave CUs idle.
    constexpr int GB2 = G == 4 ? 2 : G;
    constexpr uint64_t kCUs = 256;  // MI355X compute units
    const bool half = GB2 < G && (uint64_t)grid.x * grid.y < kCUs;
    auto go = [&](auto qc, auto oc) {
        if constexpr ((G & (G - 1)) != 0) {
            // groups of 3, 5, 6 or 7 heads: blocks of one head (two for 6), two waves per head, each
            // block copying its KV head's tiles (the thread count of a block must divide a tile's copy)
            constexpr int GBO = G % 2 == 0 ? 2 : 1;
            const dim3 g2(grid.x, grid.y * (G / GBO));
            k_attn_prefill<HD, G, GBO, decltype(qc)::value, decltype(oc)::value, WIN, 2><<<g2, 64 * GBO * 2, 0, s>>>(
                q, k, v, S, pos0, n_q, n_kv, cap, scale, o, w.win, w.n_glob, w.thr);
        } else {
            if constexpr (GB2 < G) {
                if (half) {
                    // two heads per block, four waves per head over 128-key tiles (two buffers of 64
                    // KB): eight waves, two per SIMD, and half the tiles in the longest query block's chain
                    constexpr int KS = 4;
                    const dim3 g2(grid.x, grid.y * (G / GB2));
                    k_attn_prefill<HD, G, GB2, decltype(qc)::value, decltype(oc)::value, WIN, KS, 128, 2>
                        <<<g2, 64 * GB2 * KS, 0, s>>>(q, k, v, S, pos0, n_q, n_kv, cap, scale, o, w.win, w.n_glob, w.thr);
                    return;
                }
            }
            constexpr int KS = G <= 4 ? 2 : 1;
            k_attn_prefill<HD, G, G, decltype(qc)::value, decltype(oc)::value, WIN, KS><<<grid, 64 * G * KS, 0, s>>>(
                q, k, v, S, pos0, n_q, n_kv, cap, scale, o, w.win, w.n_glob, w.thr);
        }
    };
    using T = std::true_type;
    using F = std::false_type;
    using O0 = std::integral_constant<int, 0>;
    using O1 = std::integral_constant<int, 1>;
    using O2 = std::integral_constant<int, 2>;
    if (qx2) {
        if (om == 2) go(T{}, O2{});
        else if (om == 1) go(T{}, O1{});
        else go(T{}, O0{});
    } else {
        if (om == 2) go(F{}, O2{});
        else if (om == 1) go(F{}, O1{});
        else go(F{}, O0{});
    }
}

template <int HD, int G>
static void launch_attn_prefill_g(dim3 grid, hipStream_t s, const vsl_half* q, const vsl_half* k, const vsl_half* v,
                                  uint32_t S, uint32_t pos0, uint32_t n_q, uint32_t n_kv, uint32_t cap, float scale,
                                  vsl_half* o, bool qx2, int om, const PrefillWindow& w) {
    if (w.on) launch_attn_prefill_w<HD, G, true>(grid, s, q, k, v, S, pos0, n_q, n_kv, cap, scale, o, qx2, om, w);
    else launch_attn_prefill_w<HD, G, false>(grid, s, q, k, v, S, pos0, n_q, n_kv, cap, scale, o, qx2, om, w);
}

template <int HD>
static int launch_attn_prefill(dim3 grid, hipStream_t s, const vsl_half* q, const vsl_half* k, const vsl_half* v,
                               uint32_t S, uint32_t pos0, uint32_t n_q, uint32_t n_kv, uint32_t cap, float scale,
                               vsl_half* o, bool qx2, int om, const PrefillWindow& w) {
    switch (n_q / n_kv) {
        case 1: launch_attn_prefill_g<HD, 1>(grid, s, q, k, v, S, pos0, n_q, n_kv, cap, scale, o, qx2, om, w); break;
        case 2: launch_attn_prefill_g<HD, 2>(grid, s, q, k, v, S, pos0, n_q, n_kv, cap, scale, o, qx2, om, w); break;
        case 4: launch_attn_prefill_g<HD, 4>(grid, s, q, k, v, S, pos0, n_q, n_kv, cap, scale, o, qx2, om, w); break;
        case 3: launch_attn_prefill_g<HD, 3>(grid, s, q, k, v, S, pos0, n_q, n_kv, cap, scale, o, qx2, om, w); break;
        case 5: launch_attn_prefill_g<HD, 5>(grid, s, q, k, v, S, pos0, n_q, n_kv, cap, scale, o, qx2, om, w); break;
        case 6: launch_attn_prefill_g<HD, 6>(grid, s, q, k, v, S, pos0, n_q, n_kv, cap, scale, o, qx2, om, w); break;
        case 7: launch_attn_prefill_g<HD, 7>(grid, s, q, k, v, S, pos0, n_q, n_kv, cap, scale, o, qx2, om, w); break;
        case 8: launch_attn_prefill_g<HD, 8>(grid, s, q, k, v, S, pos0, n_q, n_kv, cap, scale, o, qx2, om, w); break;
        default: return vsl_unsupported("vsl_attn_prefill: GQA ratio %u (supported 1..8)", n_q / n_kv);
    }
    return VSL_OK;
}

static int attn_prefill(const void* q, int q_dtype, const void* kcache, const void* vcache, uint32_t S, uint32_t pos0,
                        uint32_t n_q, uint32_t n_kv, uint32_t hd, uint32_t cap, float scale, void* out, int out_dtype,
                        const PrefillWindow& w, void* stream) {
    if (!q || !kcache || !vcache || !out) return vsl_invalid("vsl_attn_prefill: null pointer");
    if (S == 0) return VSL_OK;
    if (n_kv == 0 || n_q % n_kv) return vsl_invalid("vsl_attn_prefill: n_q=%u n_kv=%u", n_q, n_kv);
    if ((uint64_t)pos0 + S > cap) {
        vsl_set_error("vsl_attn_prefill: positions %u..%u exceed capacity %u", pos0, pos0 + S - 1, cap);
        return VSL_E_CAPACITY;
    }
    if ((q_dtype != VSL_DT_F16 && q_dtype != VSL_DT_F16X2) ||
        (out_dtype != VSL_DT_F16 && out_dtype != VSL_DT_F16X2 && out_dtype != VSL_DT_F16F8))
        return vsl_unsupported("vsl_attn_prefill: dtypes %d/%d", q_dtype, out_dtype);
    if (out_dtype == VSL_DT_F16F8 && (n_q * hd) % 32)
        return vsl_invalid("vsl_attn_prefill: F16F8 output needs n_q * head_dim %% 32 == 0");
    dim3 grid((S + 31) / 32, n_kv);
    hipStream_t s = static_cast<hipStream_t>(stream);
    const bool qx2 = q_dtype == VSL_DT_F16X2;
    const int om = out_dtype == VSL_DT_F16X2 ? 1 : out_dtype == VSL_DT_F16F8 ? 2 : 0;
    const vsl_half* qq = static_cast<const vsl_half*>(q);
    const vsl_half* kk = static_cast<const vsl_half*>(kcache);
    const vsl_half* vv = static_cast<const vsl_half*>(vcache);
    vsl_half* oo = static_cast<vsl_half*>(out);
    int rc;
    if (hd == 128)
        rc = launch_attn_prefill<128>(grid, s, qq, kk, vv, S, pos0, n_q, n_kv, cap, scale, oo, qx2, om, w);
    else if (hd == 64)
        rc = launch_attn_prefill<64>(grid, s, qq, kk, vv, S, pos0, n_q, n_kv, cap, scale, oo, qx2, om, w);
    else
        return vsl_unsupported("vsl_attn_prefill: head_dim %u", hd);
    if (rc) return rc;
    HIP_TRY(hipGetLastError());
    return VSL_OK;
}

extern "C" int vsl_attn_prefill(const void* q, int q_dtype, const void* kcache, const void* vcache, uint32_t S,
                                uint32_t pos0, uint32_t n_q, uint32_t n_kv, uint32_t hd, uint32_t cap, float scale,
                                void* out, int out_dtype, void* stream) {
    return attn_prefill(q, q_dtype, kcache, vcache, S, pos0, n_q, n_kv, hd, cap, scale, out, out_dtype,
                        PrefillWindow{false, 0, 0, 0}, stream);
}

extern "C" int vsl_attn_prefill_window(const void* q, int q_dtype, const void* kcache, const void* vcache, uint32_t S,
                                       uint32_t pos0, uint32_t n_q, uint32_t n_kv, uint32_t hd, uint32_t cap,
                                       float scale, void* out, int out_dtype, uint32_t window, uint32_t n_global,
                                       uint32_t threshold, void* stream) {
    if ((uint64_t)window + n_global >= 0x80000000ull)
        return vsl_invalid("vsl_attn_prefill_window: window %u + global %u too large", window, n_global);
    return attn_prefill(q, q_dtype, kcache, vcache, S, pos0, n_q, n_kv, hd, cap, scale, out, out_dtype,
                        PrefillWindow{true, window, n_global, threshold}, stream);
}
