/*
 * vsl_oracle.h -- CPU restatement of Vulkan-Symbiote-Loader's per-token forward pass.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the oracle: only tests/, the smoke() entry point of
 * __graft_entry__.py and the cpu_baseline leg of bench.py may load it.  The product (the HIP
 * backend and its host engine) never links, loads or calls it, and has no CPU fallback.
 *
 * What it restates (reference paths relative to the reference repository root):
 *   - GGUF parsing            vk_symbiote/src/GGUFLoader.cpp:625-663 (load), :847-980 (metadata,
 *                              tensor infos, read_value), :673-728 (get_model_config),
 *                              :1085-1119 (calculate_tensor_data_size), :1225-1262 (fp16->fp32),
 *                              :1121-1223 (Q4_0/Q4_1/Q8_0 dequant); enum GGUFLoader.h:18-73
 *   - token embedding          vk_symbiote/shaders/embedding_lookup.comp:29-40 (id clamped to V-1)
 *   - RMSNorm                  vk_symbiote/shaders/rms_norm.comp:24-34
 *   - RoPE (adjacent pairs)    vk_symbiote/shaders/fused_matmul_rope.comp:48-81, src/Utils.cpp:101-110
 *   - attention, GQA map       vk_symbiote/shaders/attention.comp:92,116-189
 *   - SwiGLU FFN               vk_symbiote/shaders/feed_forward.comp:21,38-62
 *   - output projection        vk_symbiote/shaders/final_linear.comp:63
 *   - layer order + residuals  architecture_design.md:308-372 (the intended Llama block; the
 *                              reference's executed code omits the residual adds and the final norm)
 *   - token loop, EOS {0,2}    vk_symbiote/src/VulkanSymbioteEngine.cpp:678-765 (:747-749)
 *   - greedy / top-k sampling  VulkanSymbioteEngine.cpp:1540-1553, 1794-1855; src/Utils.cpp:140-184
 *   - FNV-1a-64                src/Utils.cpp:9-16
 *
 * Parity status per function (what pins each one) is listed at the top of vsl_oracle.c.
 */
#ifndef VSL_ORACLE_H
#define VSL_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* tensor storage types used inside the oracle (independent of any file enum) */
enum { ORC_F32 = 0, ORC_F16 = 1 };

/* sampler modes */
enum {
    ORC_SAMPLE_GREEDY = 0,      /* VulkanSymbioteEngine::greedy_sampling: first index of the max   */
    ORC_SAMPLE_REFERENCE = 1,   /* sample_token(T>0) -> member top_k_sampling -> tokens[0]         */
    ORC_SAMPLE_TOPK_SEEDED = 2  /* Utils.cpp top_k_sampling with a Philox4x32-10 uniform           */
};

typedef struct orc_config {
    uint32_t hidden_size, num_layers, num_heads, num_kv_heads, intermediate_size, vocab_size;
    uint32_t head_dim, max_position_embeddings;
    float rope_theta, rms_eps;
} orc_config;

/* ---------------- scalar helpers ---------------- */
float orc_h2f(uint16_t h);                 /* IEEE binary16 -> binary32 (exact)                 */
uint16_t orc_f2h(float f);                 /* binary32 -> binary16, round to nearest even       */
uint64_t orc_fnv1a64(const char* s);       /* Utils.cpp:9-16 (hash_string, its own offset basis)  */
uint64_t orc_fnv1a64_basis(const char* s, uint64_t basis);
void orc_philox4x32_10(const uint32_t ctr[4], const uint32_t key[2], uint32_t out[4]);
int orc_num_threads(void);
void orc_set_num_threads(int n);

/* ---------------- GGUF ---------------- */
typedef struct orc_gguf orc_gguf;
/* returns 0 or the reference's codes: -1 open, -2 magic, -3 metadata, -4 tensor info */
int orc_gguf_open(const char* path, orc_gguf** out);
void orc_gguf_close(orc_gguf* g);
uint64_t orc_gguf_tensor_count(const orc_gguf* g);
uint64_t orc_gguf_metadata_count(const orc_gguf* g);
uint32_t orc_gguf_version(const orc_gguf* g);
uint64_t orc_gguf_data_start(const orc_gguf* g);
int orc_gguf_convention(const orc_gguf* g);   /* 0 = reference ids, 1 = ggml ids */
/* tensor info by name: returns index or -1 */
int orc_gguf_find(const orc_gguf* g, const char* name);
int orc_gguf_tensor_info(const orc_gguf* g, int idx, char* name_out, size_t name_cap,
                         uint32_t* n_dims, uint64_t dims[4], uint32_t* raw_type,
                         uint64_t* data_offset, uint64_t* data_size);
/* read tensor as fp32 (GGUFLoaderImpl::read_tensor_data semantics, Q4_0/Q4_1/Q8_0 dequantized);
 * returns element count or <0 (-20 for other quantized types) */
int64_t orc_gguf_read_f32(const orc_gguf* g, const char* name, float* out, uint64_t cap);
/* dequantize_tensor (GGUFLoader.cpp:1121-1223): raw_type in the file's convention (0 reference
 * ids 13/14/17, 1 ggml ids 2/3/8); returns floats written (fewer than n when size runs out) or -20 */
int64_t orc_dequant(const void* data, uint64_t size, uint32_t raw_type, int convention, uint64_t n, float* out);
/* metadata scalars; return 0 when found with the exact type, -1 otherwise */
int orc_gguf_get_u32(const orc_gguf* g, const char* key, uint32_t* v);
int orc_gguf_get_f32(const orc_gguf* g, const char* key, float* v);
int orc_gguf_get_str(const orc_gguf* g, const char* key, char* out, size_t cap);
/* GGUFLoader::get_model_config (GGUFLoader.cpp:673-728), plus llama.attention.layer_norm_rms_epsilon */
void orc_gguf_model_config(const orc_gguf* g, orc_config* cfg);

/* ---------------- model ---------------- */
typedef struct orc_model orc_model;
orc_model* orc_model_new(const orc_config* cfg);
void orc_model_free(orc_model* m);
/* Attach a tensor by GGUF name (data is borrowed unless copy != 0). dtype: ORC_F32 / ORC_F16 */
int orc_model_set_tensor(orc_model* m, const char* name, const void* data, int dtype, int copy);
/* Build from a GGUF file (keeps the file mapping alive inside the model). */
int orc_model_from_gguf(const char* path, orc_model** out);
void orc_model_config(const orc_model* m, orc_config* cfg);
int orc_model_check(const orc_model* m);   /* 0 if every required tensor is attached */

/* ---------------- decoding state ---------------- */
typedef struct orc_state orc_state;
/* kv_f16 != 0 stores K/V rounded to binary16 (the HBM cache format of fp16 models) */
orc_state* orc_state_new(const orc_model* m, uint32_t capacity, int kv_f16);
void orc_state_free(orc_state* s);
void orc_state_reset(orc_state* s);
/* one token at position pos (== number of cached positions); logits may be NULL */
int orc_forward(const orc_model* m, orc_state* s, uint32_t token, uint32_t pos, float* logits);
/* hidden state (after the final norm) of the last forward call, length hidden_size */
const float* orc_state_last_hidden(const orc_state* s);

/* Token loop (VulkanSymbioteEngine::generate, token-id form).  Processes the prompt, then decodes
 * up to max_new tokens.  out_tokens receives the generated ids; out_logits (optional) receives
 * max_new*vocab logits (the logits each generated token was sampled from).  stop_on_eos stops
 * after emitting 0 or 2.  Returns the number of generated tokens or <0 on error. */
int orc_generate(const orc_model* m, const uint32_t* prompt, uint32_t n_prompt, uint32_t max_new,
                 int sampler, float temperature, uint32_t top_k, uint64_t seed, int stop_on_eos,
                 int kv_f16, uint32_t* out_tokens, float* out_logits);
/* Teacher-forced logits: feeds ids[0..n-1] and stores the logits after each of the last
 * n_out positions into out (n_out*vocab). */
int orc_teacher_forced(const orc_model* m, const uint32_t* ids, uint32_t n, uint32_t n_out,
                       int kv_f16, float* out);

/* ---------------- primitives (each restates one reference op) ---------------- */
void orc_rmsnorm(const float* x, const float* gamma, uint32_t n, float eps, float* y);
void orc_rope(float* v, uint32_t n_heads, uint32_t head_dim, uint32_t pos, float theta);
/* y[N*B] (row-major [N][B]) = W[N,K] * X[K,B] with X row-major [K][B]; W dtype ORC_F32/ORC_F16 */
void orc_gemm_nt(const void* W, int wtype, uint32_t N, uint32_t K, const float* X, uint32_t B, float* Y);
/* decode attention for one query position.
 * q [n_q*hd]; K/V caches [n_kv][cap][hd] fp32; attends positions 0..len-1; out [n_q*hd] */
void orc_attention_decode(const float* q, const float* kc, const float* vc, uint32_t n_q,
                          uint32_t n_kv, uint32_t hd, uint32_t cap, uint32_t len, float scale,
                          float* out);
/* windowed mode: once len > threshold, the query at p = len - 1 attends to k < n_global and
 * k >= p - window only (threshold UINT32_MAX: dense) */
void orc_attention_decode_window(const float* q, const float* kc, const float* vc, uint32_t n_q,
                                 uint32_t n_kv, uint32_t hd, uint32_t cap, uint32_t len, float scale,
                                 uint32_t window, uint32_t n_global, uint32_t threshold, float* out);
void orc_model_set_window(orc_model* m, uint32_t window, uint32_t n_global, uint32_t threshold);
void orc_swiglu(const float* gate, const float* up, uint32_t n, float* h);
uint32_t orc_sample(const float* logits, uint32_t n, int sampler, float temperature,
                    uint32_t top_k, uint64_t seed, uint64_t step);
/* synthetic data generator: Philox4x32-10 keyed by (seed, FNV-1a-64(name)), Box-Muller.
 * out_dtype ORC_F32 or ORC_F16.  Element e uses counter block e/4, word e%4. */
void orc_fill_normal(void* out, int out_dtype, uint64_t n, uint64_t seed, const char* name,
                     float mean, float stddev);
void orc_random_ids(uint32_t* out, uint32_t n, uint32_t vocab, uint64_t seed, const char* name);

#ifdef __cplusplus
}
#endif
#endif
