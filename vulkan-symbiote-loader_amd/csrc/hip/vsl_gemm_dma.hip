// vsl_gemm_dma.hip -- prefill GEMM with direct-to-LDS loads: C[M][N] = A[M][K] * B[N][K]^T on
// v_mfma_f32_32x32x16_f16, for the shapes whose tiles fill the chip.
//
// Pipeline: BK = 32 (64 for the split 128 x 256 tile and the fp8-lo tiles) per stage, up to four LDS
// stage buffers (separate __shared__ arrays). Stage s + 3 is
// requested with global_load_lds_dwordx4 (64 lanes x 16 bytes straight into LDS, no register
// staging and no ds_write) while stage s is computed; before computing stage s a wave waits for
// its own loads of that stage (s_waitcnt vmcnt with the two younger stages still in flight) and
// the block meets at a barrier, after which every wave's part of the stage is in LDS and every
// wave has finished reading the buffer the next request overwrites. The compiler does not add
// waits of its own for loads into the other three buffers.
//
// Block = WGM x WGN waves, block tile BM x BN, wave tile (BM/WGM) x (BN/WGN) of 32 x 32 fragments:
// 2 x 2 waves of 128 x 128 (256 accumulators, one wave per SIMD) for a one-plane A; eight waves of
// 128 accumulators (two per SIMD, so one wave's MFMAs issue while the other waits on LDS reads or
// the stage barrier) for a split A, 3-6 % faster on the prefill shapes.
// LDS rows are BK = 32 halfs (64 bytes, four 16-byte chunks); chunk c of row r sits at chunk
// position c ^ ((r >> 2) & 3) of its row: a fragment read (16 lanes = 16 consecutive rows, one
// logical chunk) then touches all 16 bank groups of a 256-byte LDS cycle. Since a load instruction
// writes its 64 lanes' chunks contiguously, the swizzle is applied by choosing which global chunk
// each lane fetches.
//
// With a split A (VSL_DT_F16X2) a stage holds the hi and the lo A tiles and one B tile: both MFMAs
// of a fragment pair read the same B fragment, and B crosses L2 once (the stage grows from 24 to
// 32 KB for 128 x 256 and from 32 to 48 KB for 256 x 256, which then gets two stage buffers
// instead of four). With an fp8 lo A (VSL_DT_F16F8) a stage holds the hi tile, the B tile and a
// one-byte-per-element lo tile; the lo plane is multiplied on the fp8 matrix cores (see k_gemm_dma).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <type_traits>

#include "vsl_device.h"
#include "vsl_internal.h"

namespace {

constexpr uint32_t kKAlign = 128;  // K granularity: whole pairs of stages for every configuration

constexpr int kA1 = kGemmA1, kAX2 = kGemmAX2, kAF8 = kGemmAF8;
constexpr int kC1 = kGemmC1, kCX2 = kGemmCX2, kCF8 = kGemmCF8;

// Block tile BM x BN, BK halfs of K per stage, AP fp16 planes of A per stage (2: the hi and lo planes
// of a split A share the stage's B tile), L8: an fp8 lo plane of A after the B tile, NBUF stage
// buffers (together at most 128 KB of LDS), WGM x WGN waves of (BM / WGM) x (BN / WGN).
template <int BM_, int BN_, int BK_, int AP_, int WGM_ = 2, int WGN_ = 2, bool L8_ = false, int NBUF_ = 0,
          bool SF_ = false>
struct DmaCfg {
    static constexpr int BM = BM_, BN = BN_, BK = BK_, AP = AP_, WGM = WGM_, WGN = WGN_;
    static constexpr bool L8 = L8_;
    // SF: one fragment register set per wave (each k-step reads its own fragments and waits for them;
    // the other wave of the SIMD covers the wait), for two-wave-per-SIMD tiles short of registers
    static constexpr bool SF = SF_;
    static constexpr int NT = 64 * WGM * WGN;
    static constexpr int WM = BM / WGM, WN = BN / WGN, FM = WM / 32, FN = WN / 32;
    static constexpr int CPR = BK / 8;            // 16-byte chunks per tile row
    static constexpr int CPR8 = BK / 16;          // 16-byte chunks per row of the fp8 lo tile
    static constexpr int ACH = BM * BK / 8 / NT;  // 16-byte chunks per thread per stage, per A plane
    static constexpr int BCH = BN * BK / 8 / NT;
    static constexpr int LCH = L8 ? BM * BK / 16 / NT : 0;  // fp8 lo chunks per thread per stage
    static_assert(ACH * NT == BM * BK / 8 && BCH * NT == BN * BK / 8, "tile chunks do not divide over the threads");
    static_assert(!L8 || (LCH * NT == BM * BK / 16 && LCH >= 1), "fp8 lo chunks do not divide over the threads");
    static constexpr int L8OFF = (AP * BM + BN) * BK;          // halfs before the fp8 lo tile
    static constexpr int STAGE = L8OFF + (L8 ? BM * BK / 2 : 0);  // halfs per stage buffer
    // four stage buffers where they fit in 128 KB, else two (NBUF_ overrides; 160 KB is all of the LDS)
    static constexpr int NBUF = NBUF_ ? NBUF_ : (STAGE * 2 * 4 <= 128 * 1024 ? 4 : 2);
    static constexpr int KS = BK / 16;                  // MFMA k-steps per stage
    static_assert(STAGE * 2 * NBUF <= 160 * 1024, "stage buffers exceed the LDS");
};

__device__ __forceinline__ int d_row(int v, int lane) { return (v >> 2) * 8 + (lane >> 5) * 4 + (v & 3); }

// LDS chunk position (16-byte units) of logical chunk c of tile row r. A 256-byte LDS cycle serves
// 16 lanes of a 16-byte read, i.e. 4 rows of 64 bytes (BK 32) or 2 rows of 128 bytes (BK 64); the
// chunk index is xor-ed with the row's position among the 16 rows of a fragment read so that those
// 16 reads fall in distinct bank groups. The fp8 lo tile has rows of BK bytes: 8 rows of 32 bytes
// (CPR 2) or 4 rows of 64 bytes (CPR 4) per cycle.
template <int CPR>
__device__ __forceinline__ int chunk_pos(int r, int c) {
    if constexpr (CPR == 2) return r * 2 + (c ^ ((r >> 3) & 1));
    else if constexpr (CPR == 4) return r * 4 + (c ^ ((r >> 2) & 3));
    else return r * 8 + (c ^ ((r >> 1) & 7));
}

typedef int int8v __attribute__((ext_vector_type(8)));
typedef int int4v __attribute__((ext_vector_type(4)));

// Two fp16 values to two fp8 e4m3 bytes of v * 2^s (round to nearest even; `div` = 2^-s), into the
// low or high half of a dword. The conversion does not saturate (a magnitude past 448 becomes NaN),
// so the launcher's s keeps every |v| * 2^s of the matrix within 448.
template <bool HI_WORD>
__device__ __forceinline__ int w8_pack(int old, vsl_half a, vsl_half b, float div) {
    typedef short s2 __attribute__((ext_vector_type(2)));
    typedef _Float16 h2 __attribute__((ext_vector_type(2)));
    const h2 v = {a, b};
    s2 o = __builtin_bit_cast(s2, old);
    o = __builtin_amdgcn_cvt_scalef32_pk_fp8_f16(o, v, div, HI_WORD);
    return __builtin_bit_cast(int, o);
}

// The weight shift s of the fp8 lo product as the kernels take it: the conversion divisor 2^-s and
// the E8M0 code 127 - s of the MFMA's B scale.
struct B8Shift {
    float div;
    int e8m0;
};
inline B8Shift b8_shift(int s) { return {std::ldexp(1.0f, -s), 127 - s}; }

// SK (split K): the block's work item is (k chunk, tile); it multiplies K / ksplit of K and stores
// the fp32 partial tile to ws[chunk][M][N]; k_splitk_reduce sums the chunks in order and applies the
// epilogue (SwiGLU is not split).
//
// AM == kAF8: each k-step multiplies the hi plane on v_mfma_f32_32x32x16_f16; every 64 columns of K
// the lo plane is multiplied on v_mfma_scale_f32_32x32x64_f8f6f4 against the same B fragments
// converted to e4m3 (B * 2^s, s = the launch's weight shift) in registers, with E8M0 scales 2^-12
// and 2^-s, into the same accumulators. Operand slot j of lane group g in that MFMA is column 16 (j / 8) + 8 g + j % 8 of
// the 64: the B fragment of k-step t supplies slots 8t..8t+7, and the lo plane's byte order
// (lo8_pos) puts the A slots of a 32-column block in one 16-byte chunk per lane group.
template <class G, int EPI, int AM, int CM, bool SK>
__global__ __launch_bounds__(G::NT) void k_gemm_dma(const vsl_half* __restrict__ A, const vsl_half* __restrict__ B,
                                                       uint32_t M, uint32_t N, uint32_t K, void* __restrict__ C,
                                                       float* __restrict__ ws, uint32_t ksplit, B8Shift b8) {
    constexpr int BM = G::BM, BN = G::BN, BK = G::BK, WM = G::WM, WN = G::WN, FM = G::FM, FN = G::FN;
    constexpr int ACH = G::ACH, BCH = G::BCH, LCH = G::LCH, STAGE = G::STAGE, CPR = G::CPR, CPR8 = G::CPR8;
    constexpr int NBUF = G::NBUF, KS = G::KS;
    constexpr int AP = G::AP, NT = G::NT, WGN = G::WGN;
    constexpr bool L8 = AM == kAF8;
    static_assert(AP == (AM == kAX2 ? 2 : 1) && G::L8 == L8, "configuration / A mode mismatch");
    static_assert(!L8 || BK == 32 || BK == 64, "the fp8 lo path takes 32 or 64 columns per stage");
    static_assert(EPI != VSL_EPI_SWIGLU || FN % 2 == 0, "SwiGLU waves pair gate and up fragments");
    __shared__ __attribute__((aligned(16))) vsl_half L0[STAGE];
    __shared__ __attribute__((aligned(16))) vsl_half L1[STAGE];
    __shared__ __attribute__((aligned(16))) vsl_half L2[NBUF > 2 ? STAGE : 8];
    __shared__ __attribute__((aligned(16))) vsl_half L3[NBUF > 2 ? STAGE : 8];

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave / WGN, wn = wave % WGN;
    static_assert(!SK || EPI != VSL_EPI_SWIGLU, "SwiGLU is not split over K");
    const uint32_t ncols = EPI == VSL_EPI_SWIGLU ? BN / 2 : BN;
    const uint32_t n_m = (M + BM - 1) / BM, n_tiles = n_m * (N / ncols);
    const uint32_t n_items = SK ? n_tiles * ksplit : n_tiles;
    // XCD-aware tile order: workgroups go to the 8 XCDs round-robin by block id; each XCD takes a
    // contiguous range of work items, m fastest, so blocks sharing a B tile share an L2
    const uint32_t b = blockIdx.x, xcd = b & 7, slot = b >> 3, per = (n_items + 7) >> 3;
    const uint32_t item = xcd * per + slot;
    if (slot >= per || item >= n_items) return;
    const uint32_t kc = SK ? item / n_tiles : 0, t = SK ? item % n_tiles : item;
    const uint32_t mt = t % n_m, nt = t / n_m;
    const uint32_t m0 = mt * BM, nout0 = nt * ncols;
    const uint32_t kspan = SK ? K / ksplit : K;  // K range of this block: [kc * kspan, (kc + 1) * kspan)
    const size_t plane = (size_t)M * K;
    // the fp8 lo plane follows the hi plane (bytes)
    const vsl_half* A8 = reinterpret_cast<const vsl_half*>(reinterpret_cast<const uint8_t*>(A + plane) + (size_t)kc * kspan);
    A += (size_t)kc * kspan;
    B += (size_t)kc * kspan;

    // per-thread load sources (byte offsets without the stage's k0): load j of a stage covers
    // chunk positions j*NT + tid; position P holds row P/CPR and the logical chunk whose swizzled
    // position is P%CPR (the xor is its own inverse).
    // Byte offsets fit in 32 bits: rows * K * 2 < 2^32 is checked by the launcher.
    auto unswz = [](int P, int& r, int& c) {
        r = P / CPR;
        c = chunk_pos<CPR>(r, P % CPR) - r * CPR;
    };
    uint32_t a_off[ACH], b_off[BCH], l_off[LCH > 0 ? LCH : 1];
#pragma unroll
    for (int j = 0; j < ACH; ++j) {
        int r, c;
        unswz(j * NT + tid, r, c);
        const uint32_t gr = m0 + r < M ? m0 + r : M - 1;  // rows past M re-read row M-1 (never stored)
        a_off[j] = (gr * K + c * 8) * 2;
    }
#pragma unroll
    for (int j = 0; j < BCH; ++j) {
        int r, c;
        unswz(j * NT + tid, r, c);
        uint32_t br;
        if constexpr (EPI == VSL_EPI_SWIGLU) br = r < BN / 2 ? nout0 + r : N + nout0 + (r - BN / 2);
        else br = nout0 + r;
        b_off[j] = (br * K + c * 8) * 2;
    }
    if constexpr (L8) {
#pragma unroll
        for (int j = 0; j < LCH; ++j) {
            const int P = j * NT + tid, r = P / CPR8;
            const int c = chunk_pos<CPR8>(r, P % CPR8) - r * CPR8;
            const uint32_t gr = m0 + r < M ? m0 + r : M - 1;
            l_off[j] = gr * K + c * 16;
        }
    }
    const uint32_t nst = kspan / BK;
    // stages past the end re-load the last stage into a buffer that is not read again, keeping the
    // number of loads in flight the same at every wait
    auto issue = [&](vsl_half* L, uint32_t st) {
        const uint32_t k0 = (st < nst ? st : nst - 1) * BK;
        const vsl_half* Bp = B + k0;
#pragma unroll
        for (int p = 0; p < AP; ++p) {
            const vsl_half* Ap = A + p * plane + k0;
#pragma unroll
            for (int j = 0; j < ACH; ++j) lds_load16(Ap, a_off[j], L + p * BM * BK + (j * NT + wave * 64) * 8);
        }
#pragma unroll
        for (int j = 0; j < BCH; ++j) lds_load16(Bp, b_off[j], L + AP * BM * BK + (j * NT + wave * 64) * 8);
        if constexpr (L8) {
            const vsl_half* Lp = reinterpret_cast<const vsl_half*>(reinterpret_cast<const uint8_t*>(A8) + k0);
#pragma unroll
            for (int j = 0; j < LCH; ++j) lds_load16(Lp, l_off[j], L + G::L8OFF + (j * NT + wave * 64) * 8);
        }
    };

    float16v acc[FM][FN];
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j)
#pragma unroll
            for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.f;

    // B-tile rows of this wave's fragments; for SwiGLU the first FN/2 are gate rows, the last FN/2
    // the matching up rows
    int bt[FN];
#pragma unroll
    for (int j = 0; j < FN; ++j) {
        if constexpr (EPI == VSL_EPI_SWIGLU) bt[j] = (j < FN / 2 ? 0 : BN / 2) + wn * (WN / 2) + (j % (FN / 2)) * 32;
        else bt[j] = wn * WN + j * 32;
    }
    struct Frags {
        half8 a[AP][FM], b[FN];
    };
    auto fload = [&](Frags& f, const vsl_half* L, int ks) {
        const int lc = ks * 2 + (lane >> 5);  // logical chunk of this lane's 8 k-slots
#pragma unroll
        for (int p = 0; p < AP; ++p)
#pragma unroll
            for (int i = 0; i < FM; ++i)
                f.a[p][i] = *reinterpret_cast<const half8*>(
                    L + p * BM * BK + chunk_pos<CPR>(wm * WM + i * 32 + (lane & 31), lc) * 8);
#pragma unroll
        for (int j = 0; j < FN; ++j)
            f.b[j] = *reinterpret_cast<const half8*>(L + AP * BM * BK + chunk_pos<CPR>(bt[j] + (lane & 31), lc) * 8);
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
    // fp8 lo path: the A operand of the 64-column block (two 16-byte chunks per fragment) and the
    // e4m3 copies of the B fragments of its four k-steps
    int4v la[FM][2];
    int8v w8[FN];
    // the lo chunk of 32-column block q of this stage (lane group g = lane >> 5) into half h
    auto lload = [&](const vsl_half* L, int q, int h) {
        const uint8_t* L8p = reinterpret_cast<const uint8_t*>(L + G::L8OFF);
#pragma unroll
        for (int i = 0; i < FM; ++i)
            la[i][h] = *reinterpret_cast<const int4v*>(
                L8p + chunk_pos<CPR8>(wm * WM + i * 32 + (lane & 31), 2 * q + (lane >> 5)) * 16);
    };
    // B fragments of k-step t (0..3 within the 64-column block) -> slots 8t..8t+7
    auto wconv = [&](const Frags& f, int t) {
#pragma unroll
        for (int j = 0; j < FN; ++j) {
            int d0 = w8[j][2 * t], d1 = w8[j][2 * t + 1];
            d0 = w8_pack<false>(d0, f.b[j][0], f.b[j][1], b8.div);
            d0 = w8_pack<true>(d0, f.b[j][2], f.b[j][3], b8.div);
            d1 = w8_pack<false>(d1, f.b[j][4], f.b[j][5], b8.div);
            d1 = w8_pack<true>(d1, f.b[j][6], f.b[j][7], b8.div);
            w8[j][2 * t] = d0;
            w8[j][2 * t + 1] = d1;
        }
    };
    auto mfmas8 = [&]() {
#pragma unroll
        for (int i = 0; i < FM; ++i) {
            const int8v a8 = {la[i][0][0], la[i][0][1], la[i][0][2], la[i][0][3],
                              la[i][1][0], la[i][1][1], la[i][1][2], la[i][1][3]};
#pragma unroll
            for (int j = 0; j < FN; ++j)
                acc[i][j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a8, w8[j], acc[i][j], 0, 0, 0, 127 - 12, 0,
                                                                            b8.e8m0);
        }
    };
    constexpr int kPerStage = AP * ACH + BCH + LCH;  // loads per thread per stage
    // Stage s in buffer Lc, k-steps 0..KS-1 alternating between the fragment sets f0 / f1; k-step
    // 0 was requested during the previous stage. Each k-step requests the next one's fragments and
    // then issues its MFMAs (the reads land meanwhile). Before the last k-step's MFMAs: wait for this
    // wave's reads (Lc is fully read) and for its loads of stage s+1, meet at the barrier (every
    // wave has read Lc, every load of stage s+1 is in LDS), request stage s+NBUF into Lc, and
    // request stage s+1's first k-step from Ln. The stage count is even (K % 128 == 0 and BK <= 64)
    // and a multiple of NBUF except with four 64-column buffers, whose last round may be a pair of
    // stages; no stage is skipped or repeated. PAR is the stage's parity: with BK = 32 an fp8 lo block
    // spans an even stage and the odd stage after it.
    Frags f0, f1;
    auto step = [&](vsl_half* Lc, const vsl_half* Ln, uint32_t s, auto par) {
        constexpr int PAR = decltype(par)::value;
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
            Frags& cur = (ks & 1) ? f1 : f0;
            Frags& nxt = (ks & 1) ? f0 : f1;
            if (ks < KS - 1) {
                fload(nxt, Lc, ks + 1);
            } else {
                if constexpr (L8) {
                    // lo chunks of this stage, read late (fewer live registers) but before the
                    // barrier that lets Lc be overwritten
#pragma unroll
                    for (int q = 0; q < BK / 32; ++q) lload(Lc, q, BK == 64 ? q : PAR);
                }
                VSL_LGKM_WAIT0();
                VSL_VMCNT_WAIT((NBUF - 2) * kPerStage);
                __builtin_amdgcn_s_barrier();
                issue(Lc, s + NBUF);
                fload(nxt, Ln, 0);
            }
            __builtin_amdgcn_sched_barrier(0);
            // two waves per SIMD: the wave issuing matrix instructions goes first
            if constexpr (NT > 256) __builtin_amdgcn_s_setprio(1);
            mfmas(cur);
            if constexpr (L8) {
                const int t = BK == 64 ? ks : PAR * 2 + ks;  // k-step within the 64-column block
                wconv(cur, t);
                if (t == 3) mfmas8();
            }
            if constexpr (NT > 256) __builtin_amdgcn_s_setprio(0);
            __builtin_amdgcn_sched_barrier(0);
        }
    };
    auto step_sf = [&](vsl_half* Lc, uint32_t s, auto par) {
        constexpr int PAR = decltype(par)::value;
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
            fload(f0, Lc, ks);
            if (ks == KS - 1) {
                if constexpr (L8) {
#pragma unroll
                    for (int q = 0; q < BK / 32; ++q) lload(Lc, q, BK == 64 ? q : PAR);
                }
                VSL_LGKM_WAIT0();
                VSL_VMCNT_WAIT((NBUF - 2) * kPerStage);
                __builtin_amdgcn_s_barrier();
                issue(Lc, s + NBUF);
            }
            __builtin_amdgcn_sched_barrier(0);
            if constexpr (NT > 256) __builtin_amdgcn_s_setprio(1);
            mfmas(f0);
            if constexpr (L8) {
                const int t = BK == 64 ? ks : PAR * 2 + ks;
                wconv(f0, t);
                if (t == 3) mfmas8();
            }
            if constexpr (NT > 256) __builtin_amdgcn_s_setprio(0);
            __builtin_amdgcn_sched_barrier(0);
        }
    };
    using P0 = std::integral_constant<int, 0>;
    using P1 = std::integral_constant<int, 1>;
    issue(L0, 0);
    issue(L1, 1);
    if constexpr (NBUF == 4) {
        issue(L2, 2);
        issue(L3, 3);
    }
    VSL_VMCNT_WAIT((NBUF - 1) * kPerStage);
    __builtin_amdgcn_s_barrier();
    if constexpr (G::SF) {
        static_assert(NBUF == 2, "the single-fragment step runs two stage buffers");
        for (uint32_t s = 0; s < nst; s += 2) {
            step_sf(L0, s, P0{});
            step_sf(L1, s + 1, P1{});
        }
    } else {
        fload(f0, L0, 0);
        if constexpr (NBUF == 4) {
            uint32_t s = 0;
            for (; s + 4 <= nst; s += 4) {
                step(L0, L1, s, P0{});
                step(L1, L2, s + 1, P1{});
                step(L2, L3, s + 2, P0{});
                step(L3, L0, s + 3, P1{});
            }
            // 64-column stages in four buffers take K in multiples of 128, so a round may end with
            // one pair of stages (the requests past the last stage re-load it into buffers that are
            // not multiplied again)
            if (s < nst) {
                step(L0, L1, s, P0{});
                step(L1, L2, s + 1, P1{});
            }
        } else {
            for (uint32_t s = 0; s < nst; s += 2) {
                step(L0, L1, s, P0{});
                step(L1, L0, s + 1, P1{});
            }
        }
    }
    VSL_VMCNT_WAIT(0);  // the trailing loads land before the block's LDS is released

    // epilogue. Accumulators are read through v_accvgpr_read with an AGPR operand: with 256 of them
    // live, the epilogue's arithmetic would otherwise have the register allocator place some in
    // arch VGPRs and spill inside the main loop.
    auto rd = [](const float16v& a, int v) {
        float x;
        asm volatile("v_accvgpr_read_b32 %0, %1" : "=v"(x) : "a"(a[v]));
        return x;
    };
#pragma unroll
    for (int i = 0; i < FM; ++i) {
#pragma unroll
        for (int v = 0; v < 16; ++v) {
            const uint32_t row = m0 + wm * WM + i * 32 + d_row(v, lane);
            if (row >= M) continue;
            if constexpr (SK) {
#pragma unroll
                for (int j = 0; j < FN; ++j) {
                    const uint32_t col = nout0 + wn * WN + j * 32 + (lane & 31);
                    ws[((size_t)kc * M + row) * N + col] = rd(acc[i][j], v);
                }
            } else if constexpr (EPI == VSL_EPI_SWIGLU) {
                vsl_half* Ch = reinterpret_cast<vsl_half*>(C);
#pragma unroll
                for (int j = 0; j < FN / 2; ++j) {
                    const uint32_t col = nout0 + wn * (WN / 2) + j * 32 + (lane & 31);
                    const float h = silu(rd(acc[i][j], v)) * rd(acc[i][j + FN / 2], v);
                    if constexpr (CM == kCX2) {
                        vsl_half hi, lo;
                        split_f16(h, hi, lo);
                        Ch[(size_t)row * N + col] = hi;
                        Ch[(size_t)M * N + (size_t)row * N + col] = lo;
                    } else if constexpr (CM == kCF8) {
                        vsl_half hi;
                        uint32_t lo8;
                        split_f16_f8(h, hi, lo8);
                        Ch[(size_t)row * N + col] = hi;
                        reinterpret_cast<uint8_t*>(Ch + (size_t)M * N)[(size_t)row * N + lo8_pos(col)] = (uint8_t)lo8;
                    } else {
                        Ch[(size_t)row * N + col] = (vsl_half)h;
                    }
                }
            } else {
#pragma unroll
                for (int j = 0; j < FN; ++j) {
                    const uint32_t col = nout0 + wn * WN + j * 32 + (lane & 31);
                    const size_t o = (size_t)row * N + col;
                    const float x = rd(acc[i][j], v);
                    if constexpr (EPI == VSL_EPI_STORE_F32) reinterpret_cast<float*>(C)[o] = x;
                    else if constexpr (EPI == VSL_EPI_STORE_F16) reinterpret_cast<vsl_half*>(C)[o] = (vsl_half)x;
                    else reinterpret_cast<float*>(C)[o] += x;
                }
            }
        }
    }
}

// C = epilogue(sum over k chunks of ws[chunk]), four consecutive elements per thread, chunks added
// in order (the result does not depend on scheduling).
template <int EPI>
__global__ __launch_bounds__(256) void k_splitk_reduce(const float* __restrict__ ws, uint32_t ksplit, uint64_t MN,
                                                       void* __restrict__ C) {
    const uint64_t e = ((uint64_t)blockIdx.x * 256 + threadIdx.x) * 4;
    if (e >= MN) return;
    float4v sum = *reinterpret_cast<const float4v*>(ws + e);
#pragma unroll 8  // eight chunks' loads in flight, summed in order
    for (uint32_t k = 1; k < ksplit; ++k) sum += *reinterpret_cast<const float4v*>(ws + k * MN + e);
    if constexpr (EPI == VSL_EPI_STORE_F32) {
        *reinterpret_cast<float4v*>(static_cast<float*>(C) + e) = sum;
    } else if constexpr (EPI == VSL_EPI_STORE_F16) {
        *reinterpret_cast<half4*>(static_cast<vsl_half*>(C) + e) =
            half4{(vsl_half)sum[0], (vsl_half)sum[1], (vsl_half)sum[2], (vsl_half)sum[3]};
    } else {
        float4v* c = reinterpret_cast<float4v*>(static_cast<float*>(C) + e);
        *c = *c + sum;
    }
}

template <int BM, int BN, int TWGM = 2, int TWGN = 2, int TBK = 32, int FWGM = TWGM, int FWGN = TWGN, int FNB = 0,
          int FBK = TBK, bool FSF = false>
struct DmaPair {  // the one-plane, the split-A and the fp8-lo configuration of a block tile
    using One = DmaCfg<BM, BN, 32, 1>;
    using Two = DmaCfg<BM, BN, TBK, 2, TWGM, TWGN>;
    using F8 = DmaCfg<BM, BN, FBK, 1, FWGM, FWGN, true, FNB, FSF>;
};
// The split-A tiles run eight waves (two per SIMD, 128 accumulators each): 4 x 2 waves of 64 x 128 for
// 256 x 256, 2 x 4 waves of 64 x 64 for 128 x 256 (the one-plane tiles keep 2 x 2 waves of 128 x 128).
// The split 128 x 256 tile takes BK = 64 (two 64 KB stages, half the barriers): the K-split partials
// of a 512-row chunk, O 37.8 -> 36.6 us, down 109.9 -> 104.5 us, QKV level.
// fp8-lo tiles: 256 x 256 with BK = 64 (two 80 KB stages, all of the LDS; each row's 128-byte line
// of a stage comes in one load instruction instead of two 64-byte halves): gate/up 2048 rows 754 ->
// 690 us, 512 rows 195 -> 185 us for 2 x 2 waves of 128 x 128 against 4 x 2 waves at BK = 32. Since
// then 4 x 2 waves of 64 x 128 (two per SIMD, each raising its priority for its MFMAs) with one
// fragment register set per wave (SF; with two sets they spill): 2048 rows 688 -> 673 us, 512 rows
// level. The 128 x 256 fp8-lo tile keeps 2 x 4 waves at BK = 64 (56 KB stages) with two fragment
// sets: down 512 rows 100-102 us against 106-113 for 4 x 2, 2 x 2 and 1 x 4 waves, 102-104 for 2 x 4
// and 109-113 for 4 x 2 waves with one fragment set.
using DmaBig = DmaPair<256, 256, 4, 2, 32, 4, 2, 0, 64, true>;
using DmaMid = DmaPair<128, 256, 2, 4, 64>;
// Few-row shapes without a K split (a 128-row prompt's SwiGLU: 2 x 128 tiles of 64 rows x 64 outputs):
// 2 x 2 waves of 32 x 64 (one gate and one up fragment per wave for SwiGLU).
using DmaSmall = DmaPair<64, 128, 2, 2, 64>;
// K-split partials of widths that are a multiple of 192 but whose 128 x 256 tiles leave CUs idle (the
// QKV projection of a 512-row chunk: 6144 = 32 x 192, so 128 tiles x 2 chunks fill the 256 CUs
// where 128 x 256 gives 192 work items): 4 x 2 waves of 32 x 96, two per SIMD (against 2 x 2 waves
// of 64 x 96: hi/lo QKV with its reduce 62.9 -> 60.8 us at 512 rows, 61.3 -> 57.8 at 300).
using DmaQ = DmaPair<128, 192, 4, 2, 64, 4, 2, 0, 64>;

template <class G, int EPI>
uint32_t dma_tiles(uint32_t M, uint32_t N) {
    const uint32_t ncols = EPI == VSL_EPI_SWIGLU ? G::BN / 2 : G::BN;
    return N % ncols ? 0u : ((M + G::BM - 1) / G::BM) * (N / ncols);
}

template <class G, int EPI, int AM>
void launch_cm(uint32_t blocks, hipStream_t s, const vsl_half* a, const vsl_half* b, uint32_t M, uint32_t N,
               uint32_t K, void* C, int cm, B8Shift b8) {
    if constexpr (EPI == VSL_EPI_SWIGLU) {
        if (cm == kCX2) {
            k_gemm_dma<G, EPI, AM, kCX2, false><<<blocks, G::NT, 0, s>>>(a, b, M, N, K, C, nullptr, 1, b8);
            return;
        }
        if (cm == kCF8) {
            k_gemm_dma<G, EPI, AM, kCF8, false><<<blocks, G::NT, 0, s>>>(a, b, M, N, K, C, nullptr, 1, b8);
            return;
        }
    }
    k_gemm_dma<G, EPI, AM, kC1, false><<<blocks, G::NT, 0, s>>>(a, b, M, N, K, C, nullptr, 1, b8);
}

template <class P, int EPI>
void launch_cfg(uint32_t tiles, hipStream_t s, const vsl_half* a, const vsl_half* b, uint32_t M, uint32_t N,
                uint32_t K, void* C, int am, int cm, B8Shift b8) {
    const uint32_t blocks = ((tiles + 7) / 8) * 8;  // whole XCD ranges
    if (am == kAX2) launch_cm<typename P::Two, EPI, kAX2>(blocks, s, a, b, M, N, K, C, cm, b8);
    else if (am == kAF8) launch_cm<typename P::F8, EPI, kAF8>(blocks, s, a, b, M, N, K, C, cm, b8);
    else launch_cm<typename P::One, EPI, kA1>(blocks, s, a, b, M, N, K, C, cm, b8);
}

// split-K GEMM (partials, the epilogue's type only selects the reduce kernel)
template <class P>
void launch_splitk(uint32_t items, hipStream_t s, const vsl_half* a, const vsl_half* b, uint32_t M, uint32_t N,
                   uint32_t K, float* ws, uint32_t ksplit, int am, B8Shift b8) {
    const uint32_t blocks = ((items + 7) / 8) * 8;
    if (am == kAX2)
        k_gemm_dma<typename P::Two, VSL_EPI_STORE_F32, kAX2, kC1, true><<<blocks, P::Two::NT, 0, s>>>(
            a, b, M, N, K, nullptr, ws, ksplit, b8);
    else if (am == kAF8)
        k_gemm_dma<typename P::F8, VSL_EPI_STORE_F32, kAF8, kC1, true><<<blocks, P::F8::NT, 0, s>>>(
            a, b, M, N, K, nullptr, ws, ksplit, b8);
    else
        k_gemm_dma<typename P::One, VSL_EPI_STORE_F32, kA1, kC1, true><<<blocks, P::One::NT, 0, s>>>(
            a, b, M, N, K, nullptr, ws, ksplit, b8);
}

template <int EPI>
int launch_epi(int cfg, hipStream_t s, const vsl_half* a, const vsl_half* b, uint32_t M, uint32_t N, uint32_t K,
               void* C, int am, int cm, B8Shift b8) {
    if (cfg == 0) {
        const uint32_t t = dma_tiles<DmaBig::One, EPI>(M, N);
        if (!t) return -1;
        launch_cfg<DmaBig, EPI>(t, s, a, b, M, N, K, C, am, cm, b8);
    } else if (cfg == 1) {
        const uint32_t t = dma_tiles<DmaMid::One, EPI>(M, N);
        if (!t) return -1;
        launch_cfg<DmaMid, EPI>(t, s, a, b, M, N, K, C, am, cm, b8);
    } else {
        const uint32_t t = dma_tiles<DmaSmall::One, EPI>(M, N);
        if (!t) return -1;
        launch_cfg<DmaSmall, EPI>(t, s, a, b, M, N, K, C, am, cm, b8);
    }
    return 0;
}

}  // namespace

// Tiles of the direct-to-LDS GEMM for a shape: config 0 is 256 x 256, config 1 is 128 x 256, config 2
// is 64 x 128; 0 when the shape does not fit the configuration (N not a multiple of the tile width, K
// not of 128).
uint32_t vsl_gemm_dma_tiles(int cfg, uint32_t M, uint32_t N, uint32_t K, int epi) {
    if (K % kKAlign || K == 0) return 0;
    const uint64_t brows = epi == VSL_EPI_SWIGLU ? 2ull * N : N;
    if (((uint64_t)M * K * 2) >> 32 || (brows * K * 2) >> 32) return 0;
    const bool sw = epi == VSL_EPI_SWIGLU;
    if (cfg == 0)
        return sw ? dma_tiles<DmaBig::One, VSL_EPI_SWIGLU>(M, N) : dma_tiles<DmaBig::One, VSL_EPI_STORE_F32>(M, N);
    if (cfg == 1)
        return sw ? dma_tiles<DmaMid::One, VSL_EPI_SWIGLU>(M, N) : dma_tiles<DmaMid::One, VSL_EPI_STORE_F32>(M, N);
    return sw ? dma_tiles<DmaSmall::One, VSL_EPI_SWIGLU>(M, N) : dma_tiles<DmaSmall::One, VSL_EPI_STORE_F32>(M, N);
}

// Split-K plan for shapes whose tiles leave CUs idle: the 128 x 256 tiling with the smallest split
// in {2, 4, 8} that gives >= min_items work items and >= 512 of K per chunk; else (few rows, e.g. a
// 128-token prompt) the smallest split up to 32 with >= 128 of K per chunk that reaches min_items, or
// failing that the largest such split when it gives at least 64 items. Chunks are whole 128-wide
// stage groups. Returns the split (0: none) and the fp32 workspace bytes it needs.
uint32_t vsl_gemm_splitk_plan(uint32_t M, uint32_t N, uint32_t K, int epi, uint32_t min_items, uint64_t* ws_bytes) {
    if (ws_bytes) *ws_bytes = 0;
    if (epi == VSL_EPI_SWIGLU || N % 4) return 0;
    const uint32_t tiles = dma_tiles<DmaMid::One, VSL_EPI_STORE_F32>(M, N);
    if (!tiles || ((uint64_t)M * K * 2) >> 32 || ((uint64_t)N * K * 2) >> 32) return 0;
    auto take = [&](uint32_t ks) {
        if (ws_bytes) *ws_bytes = (uint64_t)ks * M * N * 4;
        return ks;
    };
    for (uint32_t ks : {2u, 4u, 8u})
        if (K % (ks * kKAlign) == 0 && K / ks >= 512 && tiles * ks >= min_items) return take(ks);
    uint32_t widest = 0;
    for (uint32_t ks : {2u, 4u, 8u, 16u, 32u}) {
        if (K % (ks * kKAlign) || K / ks < 128) continue;
        if (tiles * ks >= min_items) return take(ks);
        widest = ks;
    }
    return widest && tiles * widest >= 64 ? take(widest) : 0;
}

// Which tile takes the K-split partials: the 128 x 192 tile when its whole rounds of 256 work items
// cost less than the 128 x 256 tile's (tile area x rounds), else 128 x 256.
static bool splitk_narrow(uint32_t M, uint32_t N, uint32_t ksplit) {
    const uint64_t tq = dma_tiles<DmaQ::One, VSL_EPI_STORE_F32>(M, N);
    const uint64_t tm = dma_tiles<DmaMid::One, VSL_EPI_STORE_F32>(M, N);
    if (!tq || !tm) return false;
    const uint64_t rq = (tq * ksplit + 255) / 256, rm = (tm * ksplit + 255) / 256;
    return rq * 192 < rm * 256;
}

void vsl_gemm_splitk_partials(uint32_t ksplit, void* stream, const void* A, const void* B, uint32_t M, uint32_t N,
                              uint32_t K, int am, float* ws, int b8s) {
    const B8Shift b8 = b8_shift(b8s);
    const hipStream_t s = static_cast<hipStream_t>(stream);
    const vsl_half* a = static_cast<const vsl_half*>(A);
    const vsl_half* b = static_cast<const vsl_half*>(B);
    if (splitk_narrow(M, N, ksplit)) {
        const uint32_t tiles = dma_tiles<DmaQ::One, VSL_EPI_STORE_F32>(M, N);
        launch_splitk<DmaQ>(tiles * ksplit, s, a, b, M, N, K, ws, ksplit, am, b8);
        return;
    }
    const uint32_t tiles = dma_tiles<DmaMid::One, VSL_EPI_STORE_F32>(M, N);
    launch_splitk<DmaMid>(tiles * ksplit, s, a, b, M, N, K, ws, ksplit, am, b8);
}

int vsl_gemm_splitk_launch(uint32_t ksplit, void* stream, const void* A, const void* B, uint32_t M, uint32_t N,
                           uint32_t K, void* C, int epi, int am, float* ws, int b8s) {
    hipStream_t s = static_cast<hipStream_t>(stream);
    vsl_gemm_splitk_partials(ksplit, stream, A, B, M, N, K, am, ws, b8s);
    const uint64_t MN = (uint64_t)M * N;
    const uint32_t rblocks = (uint32_t)((MN / 4 + 255) / 256);
    switch (epi) {
        case VSL_EPI_STORE_F32: k_splitk_reduce<VSL_EPI_STORE_F32><<<rblocks, 256, 0, s>>>(ws, ksplit, MN, C); break;
        case VSL_EPI_STORE_F16: k_splitk_reduce<VSL_EPI_STORE_F16><<<rblocks, 256, 0, s>>>(ws, ksplit, MN, C); break;
        case VSL_EPI_RESID: k_splitk_reduce<VSL_EPI_RESID><<<rblocks, 256, 0, s>>>(ws, ksplit, MN, C); break;
        default: return -1;
    }
    return 0;
}

// Launches the direct-to-LDS GEMM; returns 0, or -1 when the shape does not fit `cfg`.
int vsl_gemm_dma_launch(int cfg, void* stream, const void* A, const void* B, uint32_t M, uint32_t N, uint32_t K,
                        void* C, int epi, int am, int cm, int b8s) {
    if (K % kKAlign || K == 0) return -1;
    const uint64_t brows = epi == VSL_EPI_SWIGLU ? 2ull * N : N;
    if (((uint64_t)M * K * 2) >> 32 || (brows * K * 2) >> 32) return -1;  // 32-bit byte offsets
    hipStream_t s = static_cast<hipStream_t>(stream);
    const vsl_half* a = static_cast<const vsl_half*>(A);
    const vsl_half* b = static_cast<const vsl_half*>(B);
    const B8Shift b8 = b8_shift(b8s);
    switch (epi) {
        case VSL_EPI_STORE_F32: return launch_epi<VSL_EPI_STORE_F32>(cfg, s, a, b, M, N, K, C, am, kC1, b8);
        case VSL_EPI_STORE_F16: return launch_epi<VSL_EPI_STORE_F16>(cfg, s, a, b, M, N, K, C, am, kC1, b8);
        case VSL_EPI_RESID: return launch_epi<VSL_EPI_RESID>(cfg, s, a, b, M, N, K, C, am, kC1, b8);
        case VSL_EPI_SWIGLU: return launch_epi<VSL_EPI_SWIGLU>(cfg, s, a, b, M, N, K, C, am, cm, b8);
        default: return -1;
    }
}

// ------------------------------------------------------------------------------------------
// Weight range of the fp8 lo product: the largest finite |w| of a matrix, and the shift s that keeps
// every |w| * 2^s within e4m3's 448.
// ------------------------------------------------------------------------------------------

// Each thread folds eight fp16 values per 16-byte load (one value per load when x is not 16-byte
// aligned) as integers: a finite binary16's magnitude bits order like its value, and an exponent field
// of all ones (infinity, NaN) is skipped. One device-scope atomic maximum per block on the float bits
// of the result (non-negative floats order like their bits; same-address atomics serialise at about
// 10 ns each, so the grid is kept to a few hundred blocks).
__global__ __launch_bounds__(256) void k_absmax_f16(const uint16_t* __restrict__ x, uint64_t n, bool vec,
                                                     uint32_t* __restrict__ out) {
    uint32_t m = 0;
    auto fold = [&](uint32_t h) {
        h &= 0x7FFFu;
        if ((h & 0x7C00u) != 0x7C00u) m = h > m ? h : m;
    };
    const uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
    const uint64_t tid = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const uint64_t nv = vec ? n / 8 : 0;
    for (uint64_t i = tid; i < nv; i += stride) {
        const uint4 v = reinterpret_cast<const uint4*>(x)[i];
        const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            fold(w[e] & 0xFFFFu);
            fold(w[e] >> 16);
        }
    }
    for (uint64_t i = nv * 8 + tid; i < n; i += stride) fold(x[i]);
#pragma unroll
    for (int off = 32; off; off >>= 1) {
        const uint32_t o = (uint32_t)__shfl_xor((int)m, off);
        m = o > m ? o : m;
    }
    __shared__ uint32_t wmax[4];
    if ((threadIdx.x & 63) == 0) wmax[threadIdx.x >> 6] = m;
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int w = 1; w < 4; ++w) m = wmax[w] > m ? wmax[w] : m;
        const float f = (float)__builtin_bit_cast(_Float16, (uint16_t)m);
        atomicMax(out, __float_as_uint(f));
    }
}

extern "C" int vsl_absmax_f16(const void* x, uint64_t n, float* max_abs, void* stream) {
    if (!x || !max_abs) return vsl_invalid("vsl_absmax_f16: null argument");
    if (reinterpret_cast<uintptr_t>(x) & 1) return vsl_invalid("vsl_absmax_f16: x must be 2-byte aligned");
    if (n == 0) return VSL_OK;
    const bool vec = (reinterpret_cast<uintptr_t>(x) & 15) == 0;
    const uint64_t items = vec ? n / 8 + 1 : n;
    const uint32_t grid = (uint32_t)std::min<uint64_t>((items + 255) / 256, 512);
    k_absmax_f16<<<grid, 256, 0, static_cast<hipStream_t>(stream)>>>(static_cast<const uint16_t*>(x), n, vec,
                                                                      reinterpret_cast<uint32_t*>(max_abs));
    HIP_TRY(hipGetLastError());
    return VSL_OK;
}

extern "C" int vsl_gemm_b8_shift(float max_abs) {
    if (!(max_abs > 0.0f) || !std::isfinite(max_abs)) return VSL_GEMM_B8_SHIFT_DEFAULT;
    int s = VSL_GEMM_B8_SHIFT_MAX;
    // exact in float: max_abs * 2^s is a power-of-two scaling of a finite value
    while (s > VSL_GEMM_B8_SHIFT_MIN && std::ldexp(max_abs, s) > 448.0f) --s;
    return s;
}
