/*
 * vsl_hip.h -- C ABI of the MI355X (gfx950) compute layer for Vulkan-Symbiote-Loader's token loop.
 *
 * This library replaces the reference's Vulkan compute column: ShaderRuntime
 * (vk_symbiote/src/ShaderRuntime.cpp, get_*_pipeline / allocate_descriptor_set /
 * dispatch_compute :1484-1541), the GLSL shaders under vk_symbiote/shaders/, the per-op VMA
 * buffers and staging round trips of VulkanSymbioteEngine.cpp (:1637-1745, :2396-2423), and the
 * GPU mirror of KVCacheManager (:64-194).  Kernels are precompiled gfx950 code objects; there is no
 * runtime shader compilation.
 *
 * Conventions
 *  - Every function returns int: 0 = OK, negative = error (VSL_E_*).  vsl_last_error() gives text.
 *  - `stream` is a hipStream_t passed as void* (NULL = the default stream).  Every launch is
 *    asynchronous on that stream.
 *  - Device pointers are owned by the caller (normally suballocated from a vsl_arena); kernels do
 *    not allocate.  Workspaces are explicit arguments.
 *  - dtype codes: VSL_DT_F32 = 0, VSL_DT_F16 = 1 (IEEE binary16).
 *  - Linear weights are row-major [out][in] ("GGUF ne0 = input dim"): y[o] = sum_i W[o*K+i] x[i]
 *    (final_linear.comp:63, feed_forward.comp:45).
 *  - Decode kernels take a device control block (vsl_ctrl) holding the current position, the
 *    sampling step and a done flag, so one captured hipGraph serves every decode step.
 */
#ifndef VSL_HIP_H
#define VSL_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
    VSL_OK = 0,
    VSL_E_INVALID = -100,     /* bad argument / shape not supported by the kernel */
    VSL_E_HIP = -101,         /* HIP runtime error */
    VSL_E_OOM = -102,         /* arena or device allocation failed */
    VSL_E_UNSUPPORTED = -103, /* dtype / layout not implemented */
    VSL_E_CAPACITY = -104     /* KV capacity or workspace too small */
};

/* VSL_DT_F16X2 -- split activations for the prefill MFMA path: an fp32 value v is held as two
 * binary16 planes, hi = fp16(v) and lo = fp16(v - hi) (hi plane first, then the lo plane of the
 * same shape), so that hi + lo carries ~22 significant bits through fp16 MFMA.
 * VSL_DT_F16F8 -- the same hi plane followed by a plane of one byte per value: the fp8 e4m3 (OCP)
 * rounding of (v - hi) * 2^12 (clamped to +-448), so that hi + lo8 * 2^-12 carries ~15 significant
 * bits for |v| <= 224 (larger values keep part of their remainder); the GEMM multiplies the lo plane
 * on the fp8 matrix cores.  Within every 32 consecutive
 * columns of a row (rows a multiple of 32 columns wide) the byte of column k sits at position k
 * with bits 3 and 4 exchanged. */
enum { VSL_DT_F32 = 0, VSL_DT_F16 = 1, VSL_DT_F16X2 = 2, VSL_DT_F16F8 = 3 };

/* Sampling modes (VulkanSymbioteEngine::sample_token, VulkanSymbioteEngine.cpp:1540-1553) */
enum {
    VSL_SAMPLE_GREEDY = 0,     /* greedy_sampling (:1794-1804): first index of the max logit        */
    VSL_SAMPLE_REFERENCE = 1,  /* T>0 through member top_k_sampling (:1806-1855), which returns its
                                  tokens[0]: the first index of the largest fp32 probability
                                  exp(l/T - max)/sum (the logit argmax unless rounding merges
                                  probabilities next to the maximum)                              */
    VSL_SAMPLE_TOPK_SEEDED = 2 /* Utils.cpp:140-172 top-k with a Philox4x32-10 uniform             */
};
/* Limit of the seeded top-k sampler (TOPK_SEEDED with T > 0): top_k >= 1 and min(top_k, V) <=
 * VSL_MAX_TOP_K (top_k > V means all of V, so every k <= V is served for V up to 262144, as the
 * reference's Utils.cpp top_k_sampling takes any k <= V); top_k = 0 and larger k return
 * VSL_E_UNSUPPORTED.  No sampler limits V. */
enum { VSL_MAX_TOP_K = 262144 };

const char* vsl_last_error(void);
int vsl_device_count(int* n);
int vsl_set_device(int device);
int vsl_device_sync(void);

/* ------------------------------------------------------------------------------------------
 * HBM arena (the FractalMemoryAllocator role, vk_symbiote/include/vk_symbiote/NomadPack.h:59-104)
 * One hipMalloc; first-fit suballocation with coalescing free list; 256-byte minimum alignment.
 * ------------------------------------------------------------------------------------------ */
typedef struct vsl_pool_stats { /* MemoryPoolStats, NomadPack.h:53-57 */
    uint64_t total_size, used_size, free_size;
    uint32_t allocation_count;
    float fragmentation_ratio;
} vsl_pool_stats;

typedef struct vsl_arena vsl_arena;
int vsl_arena_create(int device, uint64_t bytes, vsl_arena** out);
int vsl_arena_destroy(vsl_arena* a);
int vsl_arena_alloc(vsl_arena* a, uint64_t bytes, uint64_t align, void** dptr);
int vsl_arena_free(vsl_arena* a, void* dptr);
int vsl_arena_reset(vsl_arena* a);
int vsl_arena_stats(const vsl_arena* a, vsl_pool_stats* out);
void* vsl_arena_base(const vsl_arena* a);

/* ------------------------------------------------------------------------------------------
 * Packs: pinned-host staging and async upload on a side stream (NomadPack / PackManager role,
 * NomadPack.h:33-44; the reference uploads per tensor with a blocking staging copy,
 * VulkanSymbioteEngine.cpp:2051-2107).
 * ------------------------------------------------------------------------------------------ */
int vsl_host_pinned_alloc(uint64_t bytes, void** out);
int vsl_host_pinned_free(void* p);
int vsl_stream_create(void** stream);
int vsl_stream_destroy(void* stream);
int vsl_stream_sync(void* stream);
int vsl_event_create(void** ev);
int vsl_event_destroy(void* ev);
int vsl_event_record(void* ev, void* stream);
int vsl_event_sync(void* ev);
int vsl_stream_wait_event(void* stream, void* ev);
int vsl_event_elapsed_ms(void* start, void* stop, float* ms);
/* copy `bytes` from host memory (pinned for full speed) to device memory; records `done_event`
 * (may be NULL) on `stream` after the copy */
int vsl_pack_upload(void* dst_dev, const void* src_host, uint64_t bytes, void* stream, void* done_event);
int vsl_copy_d2h(void* dst_host, const void* src_dev, uint64_t bytes, void* stream);
int vsl_copy_h2d(void* dst_dev, const void* src_host, uint64_t bytes, void* stream);
int vsl_copy_d2d(void* dst_dev, const void* src_dev, uint64_t bytes, void* stream);
int vsl_memset_d(void* dst_dev, int value, uint64_t bytes, void* stream);

/* Synthetic weights on the device: Philox4x32-10 keyed by (seed, hash_string(name)) (Utils.cpp:9-16),
 * Box-Muller in fp64, rounded to the output dtype.  Same stream as the host generator. */
int vsl_fill_normal(void* dst, int dtype, uint64_t n, uint64_t seed, const char* name, float mean,
                    float stddev, void* stream);
int vsl_fill_const(void* dst, int dtype, uint64_t n, float value, void* stream);

/* ------------------------------------------------------------------------------------------
 * GGUF weight storage expanded in HBM.  Replaces the dequant-on-load of
 * GGUFLoaderImpl::read_tensor_data (vk_symbiote/src/GGUFLoader.cpp:761-793, which calls
 * dequantize_tensor :1121-1223 and returns floats for the upload): here the raw blocks are
 * uploaded and expanded on the device.
 * ------------------------------------------------------------------------------------------ */
/* storage formats (independent of either file's type ids) */
enum { VSL_WF_F32 = 0, VSL_WF_F16 = 1, VSL_WF_Q4_0 = 2, VSL_WF_Q4_1 = 3, VSL_WF_Q8_0 = 4 };
/* block layout of the quantized formats:
 *  VSL_QL_REFERENCE  files with the reference's ids (Q4_0 = 13, Q4_1 = 14, Q8_0 = 17): byte i of
 *                    the 16 nibble bytes holds elements 2i (low nibble) and 2i+1 (high nibble), as
 *                    dequantize_tensor reads them (:1163-1168); fp16 scales converted by its local
 *                    helper (:1132-1149), which drops the sign of a subnormal or zero scale
 *  VSL_QL_GGML       files with ggml's ids (2, 3, 8): byte j holds elements j (low) and j + 16
 *                    (high); scales are exact binary16
 * Each block is 32 elements: Q4_0 = fp16 d + 16 bytes, x = (nibble - 8) d; Q4_1 = fp16 d, fp16 m
 * + 16 bytes, x = nibble d + m; Q8_0 = fp16 d + 32 int8, x = q d. */
enum { VSL_QL_REFERENCE = 0, VSL_QL_GGML = 1 };
/* bytes of n elements stored in `fmt` (quantized: ceil(n / 32) whole blocks, as
 * calculate_tensor_data_size, GGUFLoader.cpp:1111-1116); 0 for an unknown format */
uint64_t vsl_weight_bytes(int fmt, uint64_t n);
/* Expand n elements in `src_fmt` (device memory, vsl_weight_bytes(src_fmt, n) bytes) into dst as
 * VSL_DT_F32 (the exact dequantized values) or VSL_DT_F16 (those values rounded to nearest even).
 * F16 / F32 sources are converted elementwise (layout ignored).  src needs 2-byte alignment (4 for
 * F32), dst 16-byte alignment; src and dst must not overlap. */
int vsl_convert_weights(const void* src, int src_fmt, int layout, uint64_t n, void* dst, int dst_dtype,
                        void* stream);

/* Resident block-quantized weight packs, multiplied block by block inside the decode GEMVs (no
 * reference counterpart: the reference expands every block to fp32 at load, GGUFLoader.cpp:1121-1223,
 * and reads 32 bits per weight per token; a pack reads 9 / 5 / 6 bits for Q8_0 / Q4_0 / Q4_1, its
 * scales held as fp32).  A pack holds a matrix
 * of `rows` x K values (K % 32 == 0) in 32-value blocks, row-major block order, as planes that each
 * start at a multiple of 256 bytes from the pack's 256-byte aligned base:
 *   VSL_DT_Q8_0  int8 values [rows][K], then fp32 scales d [rows][K/32]             w = q d
 *   VSL_DT_Q4_0  [rows][K/2] bytes (value 2j of a block in the low nibble of byte j, 2j + 1 in the
 *                high nibble), then fp32 scales d [rows][K/32]                      w = (q - 8) d
 *   VSL_DT_Q4_1  as Q4_0, then fp32 offsets m [rows][K/32]                          w = q d + m
 * The decode entry points (vsl_qkv_rope_append, vsl_gemv_residual, vsl_norm_swiglu,
 * vsl_lm_head_sample, and vsl_gemv at B = 1 with fp32 X) take these as `wdtype`; matrices stacked
 * into one operand ([Wq; Wk; Wv], [Wgate; Wup]) are consecutive rows of one pack.  Each GEMV forms
 * d * sum(q x) (+ m * sum(x)) per block in fp32. */
enum { VSL_DT_Q8_0 = 4, VSL_DT_Q4_0 = 5, VSL_DT_Q4_1 = 6 };
/* bytes of a pack of rows x K (0 for K % 32 != 0 or another dtype) */
uint64_t vsl_quant_pack_bytes(int dtype, uint32_t rows, uint32_t K);
/* n_blocks GGUF blocks (fmt VSL_WF_Q8_0 / VSL_WF_Q4_0 / VSL_WF_Q4_1 in `layout`, device memory, as
 * vsl_convert_weights reads them, same scale semantics) into blocks block0 .. block0 + n_blocks - 1
 * of the pack of the matching dtype (block b: row b / (K/32), values 32 (b % (K/32)) ..). */
int vsl_quant_pack(const void* src, int fmt, int layout, uint64_t n_blocks, void* pack, uint32_t rows, uint32_t K,
                   uint64_t block0, void* stream);
/* fp16 / fp32 weights [rows][K] into a pack, round to nearest per block: Q8_0 d = max|w| / 127;
 * Q4_0 d = -w_max / 8 (w_max the value of largest magnitude), q = clamp(round(w / d) + 8, 0, 15);
 * Q4_1 d = (max - min) / 15, m = min. */
int vsl_quantize_pack(const void* w, int wdtype, uint32_t rows, uint32_t K, int dtype, void* pack, void* stream);
/* a pack back into fp16 / fp32 weights [rows][K] (w as above, in fp32, then rounded for fp16) */
int vsl_dequant_pack(const void* pack, int dtype, uint32_t rows, uint32_t K, void* w, int wdtype, void* stream);

/* ------------------------------------------------------------------------------------------
 * Decode control block (device memory).  One per engine; read by every decode kernel.
 * ------------------------------------------------------------------------------------------ */
typedef struct vsl_ctrl {
    uint32_t pos;         /* position of the token being processed == cached positions before it */
    uint32_t step;        /* tokens sampled so far in this generation                            */
    uint32_t done;        /* 1 once max_steps tokens were sampled or EOS was hit (stop_on_eos)    */
    uint32_t stop_on_eos; /* stop after sampling 0 or 2 (VulkanSymbioteEngine.cpp:747-749)         */
    uint32_t max_steps;   /* number of tokens to sample                                          */
    uint32_t token;       /* last sampled token                                                  */
    uint32_t capacity;    /* KV capacity; decode kernels stop (done=1) rather than overflow      */
    uint32_t error;       /* nonzero when a kernel refused to run (capacity)                     */
} vsl_ctrl;

/* sampler parameters (by value) */
typedef struct vsl_sampler {
    int32_t mode;        /* VSL_SAMPLE_* ; temperature <= 0 always means greedy (sample_token :1541) */
    float temperature;
    uint32_t top_k;      /* 40 at the reference call site (VulkanSymbioteEngine.cpp:1546)         */
    uint32_t pad;
    uint64_t seed;
} vsl_sampler;

/* ------------------------------------------------------------------------------------------
 * Ops.  Each replaces one reference dispatch (shader) or a fused group of them.
 * ------------------------------------------------------------------------------------------ */

/* embedding_lookup.comp:29-40: out[t][h] = table[min(ids[t], vocab-1)][h]; out fp32 [n][d] */
int vsl_embed(const void* table, int dtype, uint32_t vocab, uint32_t d, const uint32_t* ids_dev,
              uint32_t n, float* out, void* stream);

/* rms_norm.comp:24-34 over `rows` rows: y = x / sqrt(mean(x^2)+eps) * gamma; out fp32, fp16,
 * VSL_DT_F16X2 (two planes of rows*d halfs) or VSL_DT_F16F8 (rows*d halfs, then rows*d bytes;
 * d % 32 == 0) */
int vsl_rmsnorm(const float* x, const float* gamma, uint32_t rows, uint32_t d, float eps, void* out,
                int out_dtype, void* stream);

/* GEMV / skinny GEMM (the GEMV sweep): Y[N][B] = W[N][K] * X[K][B] (X, Y row-major), fp32
 * accumulation.  W f16/f32; X, Y f16 or f32; 1 <= B <= 16; K % 8 == 0 and K <= 32768 (the limit of
 * every decode GEMV: the activation vector is staged in LDS as fp32).  f16 W with f16 X and
 * K % 512 == 0 runs on MFMA (any B, including 1); B = 1 otherwise needs fp32 X. */
int vsl_gemv(const void* W, int wdtype, uint32_t N, uint32_t K, const void* X, int xdtype, uint32_t B,
             void* Y, int ydtype, void* stream);

/* The same product for a batch of B activation vectors, each contiguous: X fp16 [B][K], Y [B][N]
 * (f16 or f32), W fp16 [N][K]; 1 <= B <= 16, K % 512 == 0.  One pass over W: B = 1 runs the decode
 * GEMV when X is 8-byte aligned and K <= 32768; whole rows streamed
 * with fp16 dot products into fp32 for 2 <= B <= 8 when X (B * K * 2 bytes) is at most 128 KB, K %
 * 1024 == 0 and X is 16-byte aligned; MFMA otherwise (W and X staged through LDS in whole-line runs
 * when K % 1024 == 0 and X is 16-byte aligned, register fragments else).  No reference
 * counterpart (the reference multiplies one vector at a time, final_linear.comp:37-85); it is the
 * batch>1 decode shape of the GEMV sweep. */
int vsl_gemv_batched(const void* W, uint32_t N, uint32_t K, const void* X, uint32_t B, void* Y, int ydtype,
                     void* stream);

/* Fused attention input stage (rms_norm.comp + attention.comp:63-108 QKV/KV-write + RoPE,
 * fused_matmul_rope.comp:48-81):
 *   n = RMSNorm(x, gamma); [q;k;v] = Wqkv n with Wqkv = [Wq; Wk; Wv] contiguous rows;
 *   RoPE (adjacent pairs, cos/sin tables [cap][hd/2]) on q and k at position ctrl->pos;
 *   q -> q_out (fp32 [n_q*hd]); k, v -> caches [n_kv][cap][hd] (kv_dtype) at ctrl->pos. */
int vsl_qkv_rope_append(const float* x, const float* gamma, float eps, const void* Wqkv, int wdtype,
                        uint32_t d, uint32_t n_q, uint32_t n_kv, uint32_t hd, const float* rope_cos,
                        const float* rope_sin, void* kcache, void* vcache, int kv_dtype, uint32_t cap,
                        float* q_out, vsl_ctrl* ctrl, void* stream);

/* Flash-decode attention (attention.comp:116-189 semantics: softmax(q.k*scale) over positions
 * 0..ctrl->pos, GQA kv_head = head*n_kv/n_q): split-KV over `nsplit` chunks with online softmax,
 * then a combine launch.  Workspace: part_o [n_q][nsplit][hd] f32, part_ml [n_q][nsplit][2] f32.
 * fp16 caches of head_dim 128 with more than 8192 positions of capacity run the scores on the
 * matrix cores (the same results to fp32 rounding; faster from about 2K attended positions). */
int vsl_attn_decode(const float* q, const void* kcache, const void* vcache, int kv_dtype, uint32_t n_q,
                    uint32_t n_kv, uint32_t hd, uint32_t cap, float scale, uint32_t nsplit, float* part_o,
                    float* part_ml, float* out, vsl_ctrl* ctrl, void* stream);

/* vsl_attn_decode with no workspace argument, for callers that cannot allocate device memory (code
 * under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).  No counterpart in the
 * reference.  The split partials go to a static device array of the library (2 MiB + 32 KiB per GPU,
 * held until the process ends): n_q * nsplit <= 4096 and head_dim <= 128, else VSL_E_CAPACITY before
 * anything is launched.  Allocates nothing.  Every call on one GPU shares that array, so calls that
 * overlap on one GPU (concurrent streams, threads) race; calls ordered on one stream do not.  Results
 * are those of vsl_attn_decode bit for bit. */
int vsl_attn_decode_noalloc(const float* q, const void* kcache, const void* vcache, int kv_dtype, uint32_t n_q,
                            uint32_t n_kv, uint32_t hd, uint32_t cap, float scale, uint32_t nsplit, float* out,
                            vsl_ctrl* ctrl, void* stream);

/* Windowed long-context mode (the reference's use_sparse_attention, Common.h:70-75, switched on
 * above `seq_len > 8192` at VulkanSymbioteEngine.cpp:788; sparse_attention.comp:77-100 sliding
 * window + global tokens).  With p = ctrl->pos: while p + 1 <= threshold the query attends to every
 * key 0..p (as vsl_attn_decode); past it, to the keys k < n_global and p - window <= k <= p only.
 * Replaces sparse_attention_with_weights (VulkanSymbioteEngine.cpp:2592-2724), whose shader drops
 * the global tokens and zeroes scores past index 512; those defects are not reproduced.
 * window + n_global < 2^31. */
int vsl_attn_decode_window(const float* q, const void* kcache, const void* vcache, int kv_dtype, uint32_t n_q,
                           uint32_t n_kv, uint32_t hd, uint32_t cap, float scale, uint32_t nsplit, float* part_o,
                           float* part_ml, float* out, vsl_ctrl* ctrl, uint32_t window, uint32_t n_global,
                           uint32_t threshold, void* stream);

/* y[N] += W[N][K] x[K]  (O projection / FFN down projection with the residual add fused);
 * K % 8 == 0, K <= 32768 */
int vsl_gemv_residual(const void* W, int wdtype, uint32_t N, uint32_t K, const float* x, float* resid,
                      vsl_ctrl* ctrl, void* stream);

/* feed_forward.comp:21,38-51 fused with the FFN RMSNorm:
 *   m = RMSNorm(x, gamma); h = silu(Wgate m) * (Wup m), with Wgu = [Wgate; Wup] contiguous rows;
 *   h fp32 [F] */
int vsl_norm_swiglu(const float* x, const float* gamma, float eps, const void* Wgu, int wdtype,
                    uint32_t d, uint32_t F, float* h_out, vsl_ctrl* ctrl, void* stream);

/* Output stage (final norm + final_linear.comp + sample_token) for one position:
 *   f = RMSNorm(x, gamma) (gamma may be NULL: no final norm); logits = W f (fp32 [V]);
 *   greedy: per-block argmax fused into the GEMV, reduced by a second launch;
 *   reference and top-k modes (T > 0): the GEMV writes logits and a sampling launch follows
 *   (top-k limit: min(top_k, V) <= VSL_MAX_TOP_K; otherwise VSL_E_UNSUPPORTED before any launch).
 *   The sampled token is written to tokens[ctrl->step]; then x <- embed[token] (the next step's
 *   embedding_lookup), ctrl->pos += 1, ctrl->step += 1, and done is set on max_steps / EOS.
 *   Workspace: ws_val/ws_idx >= vsl_lm_head_ws_blocks() entries. */
int vsl_lm_head_sample(const float* gamma, float eps, const void* W, int wdtype, uint32_t V, uint32_t d,
                       float* x, const void* embed, int embed_dtype, float* logits, vsl_sampler sampler,
                       float* ws_val, uint32_t* ws_idx, uint32_t* tokens, vsl_ctrl* ctrl, void* stream);
uint32_t vsl_lm_head_ws_blocks(void);

/* Sample one token from fp32 logits already in memory (no bookkeeping): the samplers alone,
 * exposed for the sampler parity tests.  out: one u32.  Sampler limits as above. */
int vsl_sample_logits(const float* logits, uint32_t V, vsl_sampler sampler, uint64_t step,
                      uint32_t* out, void* stream);

/* Host-side reset of the control block (device memory) for a new generation. */
int vsl_ctrl_reset(vsl_ctrl* ctrl, uint32_t pos, uint32_t max_steps, uint32_t stop_on_eos,
                   uint32_t capacity, void* stream);

/* ------------------------------------------------------------------------------------------
 * Prefill (S positions at once): fp16 MFMA GEMMs and flash attention.
 * ------------------------------------------------------------------------------------------ */
/* C[M][N] (+)= A[M][K] * B[N][K]^T, fp16 inputs, fp32 accumulate.  epilogue:
 *   VSL_EPI_STORE_F32 (C f32), VSL_EPI_STORE_F16 (C f16), VSL_EPI_RESID (C f32 +=),
 *   VSL_EPI_SWIGLU (B = [Wgate; Wup], N = F: C f16 = silu(A Wg^T) * (A Wu^T)).
 * Flags or'ed into `epilogue`: VSL_GEMM_A_X2 (A is VSL_DT_F16X2: two MFMAs per tile, hi and lo),
 * VSL_GEMM_C_X2 (SwiGLU output written as VSL_DT_F16X2), VSL_GEMM_A_F8 (A is VSL_DT_F16F8: the hi
 * plane on fp16 MFMA, the lo plane on fp8 MFMA against B rounded to e4m3 as B * 2^s, into the same
 * fp32 accumulators), VSL_GEMM_C_F8 (SwiGLU output written as VSL_DT_F16F8).  The F8 forms need
 * N % 256 == 0 (N % 128 == 0 for SwiGLU) and K % 128 == 0, else VSL_E_UNSUPPORTED.
 * The weight shift s of the fp8 lo product is or'ed in as VSL_GEMM_B8_SHIFT(s), -16 <= s <= 30
 * (without it s = 6).  e4m3 holds magnitudes up to 448 and the conversion does not saturate, so
 * every |B| * 2^s must be <= 448: vsl_gemm_b8_shift gives the largest such s for a matrix's
 * largest magnitude (vsl_absmax_f16), which also keeps the small weights out of e4m3's subnormal
 * range as far as the large ones allow. */
enum { VSL_EPI_STORE_F32 = 0, VSL_EPI_STORE_F16 = 1, VSL_EPI_RESID = 2, VSL_EPI_SWIGLU = 3 };
enum { VSL_GEMM_A_X2 = 0x100, VSL_GEMM_C_X2 = 0x200, VSL_GEMM_A_F8 = 0x400, VSL_GEMM_C_F8 = 0x800 };
#define VSL_GEMM_B8_SHIFT(s) ((int)((((s) + 128) & 0xFF) << 16))
enum { VSL_GEMM_B8_SHIFT_MIN = -16, VSL_GEMM_B8_SHIFT_MAX = 30, VSL_GEMM_B8_SHIFT_DEFAULT = 6 };
/* The largest s in [VSL_GEMM_B8_SHIFT_MIN, VSL_GEMM_B8_SHIFT_MAX] with max_abs * 2^s <= 448 (e4m3's
 * largest finite value); VSL_GEMM_B8_SHIFT_DEFAULT for max_abs 0 or not finite. */
int vsl_gemm_b8_shift(float max_abs);
/* The largest finite |x| over n fp16 values (NaN and infinities skipped) folded into *max_abs (a
 * device float, which the caller sets to 0 first or which holds a previous maximum to extend) by
 * device-scope atomic maxima. */
int vsl_absmax_f16(const void* x, uint64_t n, float* max_abs, void* stream);
int vsl_gemm_f16(const void* A, const void* B, uint32_t M, uint32_t N, uint32_t K, void* C, int epilogue,
                 void* stream);
/* The same with an fp32 workspace (16-byte aligned): shapes whose output tiles would leave CUs idle
 * (e.g. M = 512 against N = 4096) are split over K, the partials summed in a fixed order by a second
 * launch that applies the epilogue (not for VSL_EPI_SWIGLU).  vsl_gemm_f16_ws_bytes gives the bytes a
 * shape uses (0: no split, the workspace is not touched); with less than that the call runs
 * unsplit. */
int vsl_gemm_f16_ws(const void* A, const void* B, uint32_t M, uint32_t N, uint32_t K, void* C, int epilogue,
                    void* workspace, uint64_t ws_bytes, void* stream);
uint64_t vsl_gemm_f16_ws_bytes(uint32_t M, uint32_t N, uint32_t K, int epilogue);
/* 1 when vsl_gemm_f16_ws (with vsl_gemm_f16_ws_bytes of workspace) runs this shape on the
 * direct-to-LDS kernel -- the one with the F8 forms -- through whole tiles that cover three quarters
 * of the CUs (192 tiles of 256 x 256 or 128 x 256), or through a K split: the smallest split giving
 * 192 work items where K allows one, else the widest split K allows when that gives at least 64
 * items (few-row shapes such as a 128-row prompt against N = 2048); 0 when it would take the
 * register-staged kernel instead (an F8 form then forces the direct-to-LDS tiles at lower occupancy,
 * e.g. a 128-row SwiGLU on 64 tiles). */
int vsl_gemm_f16_direct(uint32_t M, uint32_t N, uint32_t K, int epilogue);

/* Q/K/V split of a prefill QKV GEMM output (f32 [S][(n_q+2 n_kv) hd]) with RoPE at positions
 * pos0..pos0+S-1: q -> q_out [S][n_q][hd] (q_dtype VSL_DT_F16 or VSL_DT_F16X2), k/v -> caches at
 * pos0+s. */
int vsl_rope_split_append(const float* qkv, uint32_t S, uint32_t n_q, uint32_t n_kv, uint32_t hd,
                          uint32_t pos0, const float* rope_cos, const float* rope_sin, void* q_out, int q_dtype,
                          void* kcache, void* vcache, int kv_dtype, uint32_t cap, void* stream);

/* The attention stage's entry for S prompt rows (forward_layer_with_weights,
 * VulkanSymbioteEngine.cpp:777-806, normed -> attention_with_weights): the QKV projection of A
 * [S][K] against Wqkv [(n_q+2 n_kv) hd][K] followed by vsl_rope_split_append.  `a_flags` is 0,
 * VSL_GEMM_A_X2 or VSL_GEMM_A_F8 (with an optional VSL_GEMM_B8_SHIFT).  When the shape splits over K (workspace as for vsl_gemm_f16_ws), the partials are
 * summed, rotated and stored by one launch and qkv is not touched; otherwise qkv (f32 [S][(n_q+2 n_kv)
 * hd]) receives the projection first.  Checks (capacity, dtypes) happen before anything is launched. */
int vsl_gemm_f16_qkv_rope_append(const void* A, const void* Wqkv, uint32_t S, uint32_t K, int a_flags,
                                 uint32_t n_q, uint32_t n_kv, uint32_t hd, uint32_t pos0, const float* rope_cos,
                                 const float* rope_sin, void* q_out, int q_dtype, void* kcache, void* vcache,
                                 int kv_dtype, uint32_t cap, float* qkv, void* workspace, uint64_t ws_bytes,
                                 void* stream);

/* A residual projection and the RMSNorm that starts the next stage (forward_layer_with_weights,
 * VulkanSymbioteEngine.cpp:777-806: the attention output feeds the FFN's norm, the FFN output the
 * next layer's attention norm): x [M][N] f32 += A [M][K] B [N][K]^T, then xn = rmsnorm(x) * gamma as
 * vsl_rmsnorm (xn_dtype F16, F16X2, F16F8 or F32; `a_flags` as for the QKV entry).  When the shape splits over K, one launch sums the
 * partials in order, adds them to x and normalizes the rows; otherwise the residual GEMM is followed
 * by vsl_rmsnorm. */
int vsl_gemm_f16_resid_rmsnorm(const void* A, const void* B, uint32_t M, uint32_t N, uint32_t K, int a_flags,
                               float* x, const float* gamma, float eps, void* xn, int xn_dtype, void* workspace,
                               uint64_t ws_bytes, void* stream);

/* Causal prefill attention for S queries at positions pos0..pos0+S-1 against cache positions
 * 0..pos0+s: q [S][n_q][hd] (q_dtype F16 or F16X2), caches f16 [n_kv][cap][hd],
 * out [S][n_q*hd] (out_dtype F16, F16X2 or F16F8).  With F16X2 q the probabilities are split as well. */
int vsl_attn_prefill(const void* q, int q_dtype, const void* kcache, const void* vcache, uint32_t S,
                     uint32_t pos0, uint32_t n_q, uint32_t n_kv, uint32_t hd, uint32_t cap, float scale,
                     void* out, int out_dtype, void* stream);
/* The same with the windowed mode of vsl_attn_decode_window applied per row: the row at position
 * p attends to 0..p while p + 1 <= threshold, else to k < n_global and p - window <= k <= p. */
int vsl_attn_prefill_window(const void* q, int q_dtype, const void* kcache, const void* vcache, uint32_t S,
                            uint32_t pos0, uint32_t n_q, uint32_t n_kv, uint32_t hd, uint32_t cap, float scale,
                            void* out, int out_dtype, uint32_t window, uint32_t n_global, uint32_t threshold,
                            void* stream);

/* ------------------------------------------------------------------------------------------
 * hipGraph helpers (each decode step is captured once and replayed).
 * ------------------------------------------------------------------------------------------ */
typedef struct vsl_graph vsl_graph;
int vsl_graph_begin(void* stream);
int vsl_graph_end(void* stream, vsl_graph** out);
int vsl_graph_launch(vsl_graph* g, void* stream);
int vsl_graph_destroy(vsl_graph* g);

#ifdef __cplusplus
}
#endif
#endif
