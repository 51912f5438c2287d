/*
 * vsl_engine.h -- C ABI of the MI355X engine (the token loop behind
 * VulkanSymbioteEngine::generate(), vk_symbiote/src/VulkanSymbioteEngine.cpp:678-765).
 *
 * The reference exposes only a C++ class (vk_symbiote/include/vk_symbiote/VulkanSymbioteEngine.h:72-118)
 * and has no FFI.  These entry points are what a foreign binding of that class needs: open a model
 * (constructor, :74), generate from token ids (the additive token-id form of generate, :86),
 * generate from text (:86), config() (:90), run_benchmark (:98), get_vram_stats (:112),
 * clear_kv_cache / get_kv_cache_memory_usage (:116-117), and GGUFLoader's model-file format
 * (write_synthetic_gguf produces files the reference's loader layout reads).
 * All functions return 0 on success and a negative code on failure; vsl_engine_last_error()
 * gives the message of the calling thread's last failure.
 */
#ifndef VSL_ENGINE_H
#define VSL_ENGINE_H

#include <stddef.h>
#include <stdint.h>

#include "vsl_hip.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct vsl_engine vsl_engine;

/* ModelConfig (Common.h:56-76) subset that defines a Llama-style decoder */
typedef struct vsl_model_spec {
    uint32_t hidden_size, num_layers, num_heads, num_kv_heads, intermediate_size, vocab_size;
    uint32_t max_position_embeddings;
    float rope_theta, rms_eps;
    float init_std;    /* synthetic weights only: N(0, init_std) */
    uint32_t dtype;    /* storage of the linear weights: VSL_WF_F32 (== VSL_DT_F32) or VSL_WF_F16
                          (== VSL_DT_F16); VSL_WF_Q4_0 / Q4_1 / Q8_0: vsl_write_synthetic_gguf stores
                          every 2-D weight block-quantized from the fp32 draws, and
                          vsl_engine_open_synthetic quantizes fp16 draws of every linear weight on the
                          device into resident packs (vsl_quantize_pack; needs quant_decode), whose
                          values the expanded packs hold in fp16 (fp32 with dequant_f32) */
    uint32_t head_dim; /* filled by vsl_engine_get_config; ignored on input */
} vsl_model_spec;

typedef struct vsl_engine_options {
    int32_t device;
    uint32_t kv_capacity;    /* 0 = min(context length, 4096) */
    uint32_t use_graph;      /* 1 = capture each decode step as a hipGraph (default) */
    uint32_t prefill_chunk;  /* 0 = 2048 */
    uint32_t attn_splits;    /* 0 = automatic */
    uint32_t batched_prefill;/* 1 = MFMA prefill for fp16 models (default) */
    uint32_t prefill_split;  /* prefill activations carried as hi/lo fp16 pairs: bit 0 QKV input, bit 1
                                attention q/probabilities, bit 2 O input, bit 3 gate/up input, bit 4
                                down input; vsl_engine_default_options sets all five */
    uint32_t dequant_f32;    /* block-quantized GGUF weights expand to fp32 packs (the exact values of
                                dequantize_tensor, GGUFLoader.cpp:1121-1223) instead of fp16 packs */
    uint32_t sparse_attention;  /* 1 = windowed long-context mode (use_sparse_attention, Common.h:70-75):
                                   a query at position p with p + 1 > sparse_threshold attends to the
                                   first sparse_global keys and the sparse_window keys before it only */
    uint32_t sparse_window;     /* vsl_engine_default_options: 512 */
    uint32_t sparse_global;     /* 16 */
    uint32_t sparse_threshold;  /* 8192 (the reference's seq_len > 8192, VulkanSymbioteEngine.cpp:788) */
    uint32_t prefill_lo8;       /* split stages whose lo part is fp8 (VSL_DT_F16F8, the lo plane on the fp8
                                   matrix cores): bit 0 QKV input, bit 2 O input, bit 3 gate/up input,
                                   bit 4 down input;
                                   taken where the shapes allow it (d, F and the QKV width multiples of
                                   256), else the fp16 lo plane; vsl_engine_default_options sets 0x1C */
    uint32_t quant_decode;      /* 1 (default): block-quantized weights also stay resident as blocks
                                   (vsl_quant_pack) and the decode GEMVs read those; the prompt pass
                                   uses the expanded packs */
} vsl_engine_options;

typedef struct vsl_gen_params {
    int32_t mode;          /* VSL_SAMPLE_* */
    float temperature;     /* <= 0 means greedy */
    uint32_t top_k;        /* VSL_SAMPLE_TOPK_SEEDED: 40 at the reference call site */
    uint32_t stop_on_eos;  /* stop after sampling 0 or 2 (VulkanSymbioteEngine.cpp:747-749) */
    uint64_t seed;
} vsl_gen_params;

typedef struct vsl_gen_stats {
    uint32_t prompt_tokens, generated_tokens, kv_positions, pad;
    double prefill_ms, decode_ms;
} vsl_gen_stats;

void vsl_engine_default_options(vsl_engine_options* o);
const char* vsl_engine_last_error(void);

int vsl_engine_open(const char* gguf_path, const vsl_engine_options* opt, vsl_engine** out);
int vsl_engine_open_synthetic(const vsl_model_spec* spec, uint64_t seed, const vsl_engine_options* opt,
                              vsl_engine** out);
int vsl_engine_close(vsl_engine* e);

/* Token-id generation.  out_tokens holds max_new entries; out_logits (nullable) holds
 * max_new * vocab floats: the logits each generated token was sampled from.  *n_out receives the
 * number of generated tokens. */
int vsl_engine_generate_ids(vsl_engine* e, const uint32_t* prompt, uint32_t n_prompt, uint32_t max_new,
                            const vsl_gen_params* params, uint32_t* out_tokens, float* out_logits, uint32_t* n_out);
/* Teacher-forced generation (parity checks): as vsl_engine_generate_ids, but step t + 1 takes forced[t]
 * as its input instead of the token sampled at step t (n_forced >= max_new - 1), and EOS does not stop
 * the run.  out_tokens receives the sampled tokens, out_logits each step's logits, so that every step
 * can be compared with another implementation fed the same token history.  No reference counterpart
 * (the reference's generate always feeds back its own samples, VulkanSymbioteEngine.cpp:730-760). */
int vsl_engine_generate_forced(vsl_engine* e, const uint32_t* prompt, uint32_t n_prompt, const uint32_t* forced,
                               uint32_t n_forced, uint32_t max_new, const vsl_gen_params* params, uint32_t* out_tokens,
                               float* out_logits, uint32_t* n_out);
/* generate(prompt, max_tokens, temperature): text in, prompt + decode({id}) of each generated token out
 * (NUL-terminated), with the tokenizer of the model file (the byte fallback for synthetic engines) */
int vsl_engine_generate_text(vsl_engine* e, const char* prompt, uint32_t max_tokens, float temperature, char* out,
                             uint64_t out_cap, uint64_t* out_len);

/* Split form of generate_ids (prefill timed apart from decode): begin runs the prompt and samples
 * the first token; decode enqueues up to n decode steps without waiting (*issued receives how many);
 * finish waits, then copies the generated tokens (max_new entries) and sets *n_out. */
int vsl_engine_begin(vsl_engine* e, const uint32_t* prompt, uint32_t n_prompt, uint32_t max_new,
                     const vsl_gen_params* params);
int vsl_engine_decode(vsl_engine* e, uint32_t n, uint32_t* issued);
int vsl_engine_sync(vsl_engine* e);
int vsl_engine_finish(vsl_engine* e, uint32_t* out_tokens, uint32_t* n_out);
/* Average device time (ms) of one launch of a decode op, HIP events on the engine's stream, every
 * layer visited per round: 0 qkv+rope+kv-append, 1 attention, 2 o-proj+residual,
 * 3 ffn-norm+gate/up+swiglu, 4 down-proj+residual, 5 final-norm+lm_head+argmax. */
int vsl_engine_time_op(vsl_engine* e, int op, uint32_t iterations, double* avg_ms);

int vsl_engine_get_config(vsl_engine* e, vsl_model_spec* out);
int vsl_engine_last_stats(vsl_engine* e, vsl_gen_stats* out);
int vsl_engine_vram_stats(vsl_engine* e, vsl_pool_stats* out);
int vsl_engine_kv_bytes(vsl_engine* e, uint64_t* out);
int vsl_engine_weight_bytes(vsl_engine* e, uint64_t* out);
int vsl_engine_clear_kv(vsl_engine* e);
/* run_benchmark(warmup, tokens, iterations) -> average / min / max decode tok/s */
int vsl_engine_benchmark(vsl_engine* e, uint32_t warmup, uint32_t tokens, uint32_t iterations, double* avg_tps,
                         double* min_tps, double* max_tps);
/* device -> host copy of one resident pack (GGUF tensor name); *dtype_out = VSL_DT_* */
int vsl_engine_read_tensor(vsl_engine* e, const char* name, void* dst, uint64_t bytes, int* dtype_out);

/* Pack metadata (PackMetadata, NomadPack.h:33-44, as GGUFLoader::generate_packs fills it,
 * GGUFLoader.cpp:730-751: one pack per tensor, pack_id = std::hash(name), type by name :1302-1315,
 * layer from "blk.<n>" :1264-1272, priority :1279-1300).  For an engine's packs also where each one
 * lives: device pointer, resident bytes (after any expansion), dtype and tier (VRAM_HOT = 0). */
typedef struct vsl_pack_info {
    uint64_t pack_id;
    int32_t type;           /* PackType: 0..3 attention Q/K/V/O, 4 gate (and up), 6 down, 7 norm,
                               10 embedding, 11 head, 255 unknown */
    uint32_t layer_idx, head_idx, alignment;
    uint64_t compressed_size, decompressed_size, file_offset;
    float base_priority;
    int32_t tier;           /* engine packs: MemoryTier; GGUF packs: -1 */
    int32_t dtype;          /* engine packs: VSL_DT_*; GGUF packs: -1 */
    uint32_t n_dimensions;
    uint64_t resident_bytes; /* engine packs: bytes in HBM; GGUF packs: 0 */
    void* device_ptr;        /* engine packs: the pack's HBM address; GGUF packs: NULL */
} vsl_pack_info;
int vsl_engine_pack_count(vsl_engine* e, uint64_t* n);
/* name receives the tensor name (NUL-terminated, truncated to name_cap) */
int vsl_engine_pack(vsl_engine* e, uint64_t idx, vsl_pack_info* out, char* name, uint64_t name_cap);

/* GGUF writer: synthetic Llama-style model with the reference's tensor names.
 * convention 0 = the reference's tensor-type ids (F32 6, F16 48, Q4_0 13, Q4_1 14, Q8_0 17) and
 * block layout, 1 = ggml ids (F32 0, F16 1, Q4_0 2, Q4_1 3, Q8_0 8) and ggml's block layout. */
int vsl_write_synthetic_gguf(const char* path, const vsl_model_spec* spec, uint64_t seed, int convention);
/* the same with a vocabulary: n_tokens strings (tokens[i], token_lens[i] bytes each, may hold any
 * byte) written as the array "tokenizer.ggml.tokens", or with keyed = 1 as one string key
 * "tokenizer.ggml.tokens.<i>" per token (the layout the reference's Tokenizer::from_gguf scans for,
 * Tokenizer.cpp:55-74) */
int vsl_write_synthetic_gguf_vocab(const char* path, const vsl_model_spec* spec, uint64_t seed, int convention,
                                   const char* const* tokens, const uint64_t* token_lens, uint32_t n_tokens,
                                   int keyed);
/* the host synthetic generator (same stream as vsl_fill_normal) */
int vsl_synthetic_fill_host(void* out, int dtype, uint64_t n, uint64_t seed, const char* name, float mean,
                            float stddev);

/* GGUFLoader (GGUFLoader.h:265-333): load / get_model_config / get_tensor / read_tensor_data.
 * vsl_gguf_open returns the reference's codes: -1 open, -2 magic, -3 metadata, -4 tensor info. */
typedef struct vsl_gguf vsl_gguf;
int vsl_gguf_open(const char* path, vsl_gguf** out);
int vsl_gguf_close(vsl_gguf* g);
int vsl_gguf_info(vsl_gguf* g, uint64_t* tensor_count, uint64_t* metadata_count, uint32_t* version, int* convention,
                  uint64_t* data_start);
int vsl_gguf_model_config(vsl_gguf* g, vsl_model_spec* out);
/* -30 when the tensor does not exist */
int vsl_gguf_tensor(vsl_gguf* g, const char* name, uint64_t* data_offset, uint64_t* data_size, uint32_t* raw_type,
                    uint32_t* n_dims, uint64_t dims[4]);
/* GGUFLoader::generate_packs: the packs of every tensor, in file order */
int vsl_gguf_pack_count(vsl_gguf* g, uint64_t* n);
int vsl_gguf_pack(vsl_gguf* g, uint64_t idx, vsl_pack_info* out, char* name, uint64_t name_cap);
/* returns the element count, or the reference's read codes (-11 read, -12 type, -20 quantized, -30 missing);
 * Q4_0 / Q4_1 / Q8_0 tensors are dequantized (dequantize_tensor, GGUFLoader.cpp:1121-1223) */
int64_t vsl_gguf_read_f32(vsl_gguf* g, const char* name, float* out, uint64_t cap);

/* Tokenizer (vk_symbiote/include/vk_symbiote/Tokenizer.h:7-22): the vocabulary of a GGUF file
 * (array "tokenizer.ggml.tokens", else keys "tokenizer.ggml.tokens.<id>"), or the 256-byte fallback
 * when gguf_path is NULL or the file has neither (the reference also falls back on an unreadable
 * file).  encode / decode follow Tokenizer.cpp:131-198: whitespace-split words, a word found in the
 * vocabulary is one id, else one id per byte (found, or (signed byte * 31) % 31000 + 1000); an empty
 * text gives [0]; decode joins vocab[id % vocab_size] with single spaces.
 * vsl_tokenizer_encode writes min(*n_out, cap) ids and sets *n_out to the full count;
 * vsl_tokenizer_decode writes at most cap bytes (no terminator) and sets *len_out to the full
 * length.  source: 0 bytes, 1 array, 2 keys. */
typedef struct vsl_tokenizer vsl_tokenizer;
int vsl_tokenizer_open(const char* gguf_path, vsl_tokenizer** out);
int vsl_tokenizer_close(vsl_tokenizer* t);
int vsl_tokenizer_info(vsl_tokenizer* t, uint32_t* vocab_size, int* source);
int vsl_tokenizer_encode(vsl_tokenizer* t, const char* text, uint64_t text_len, uint32_t* ids, uint64_t cap,
                         uint64_t* n_out);
int vsl_tokenizer_decode(vsl_tokenizer* t, const uint32_t* ids, uint64_t n, char* out, uint64_t cap,
                         uint64_t* len_out);

/* ConfigManager (ConfigManager.h:133-270): parse CLI args / a TOML file into the singleton and read
 * the fields the engine uses.  enable_gpu is 0 after --disable-gpu; opening an engine then fails. */
int vsl_config_load_args(int argc, const char* const* argv);
int vsl_config_load_file(const char* path);
int vsl_config_save_file(const char* path);
int vsl_config_reset(void);
int vsl_config_get(int* enable_gpu, int* device, uint32_t* kv_capacity, uint64_t* seed, float* vram_budget_gb);

#ifdef __cplusplus
}
#endif
#endif
