// engine_capi.cpp -- extern "C" wrapper of VulkanSymbioteEngine / GGUF writer / ConfigManager.
#include <algorithm>
#include <cstring>
#include <memory>
#include <string>
#include <vector>

#include "ConfigManager.h"
#include "VulkanSymbioteEngine.h"
#include "vsl_engine.h"

using namespace vk_symbiote;

struct vsl_engine {
    std::unique_ptr<VulkanSymbioteEngine> impl;
};

static thread_local std::string g_engine_error;

static int fail(int code, const std::string& msg) {
    g_engine_error = msg;
    return code;
}

extern "C" const char* vsl_engine_last_error(void) { return g_engine_error.c_str(); }

extern "C" void vsl_engine_default_options(vsl_engine_options* o) {
    if (!o) return;
    std::memset(o, 0, sizeof(*o));
    o->use_graph = 1;
    o->batched_prefill = 1;
    o->prefill_split = EngineOptions::kPrefillSplitAll;
    o->prefill_lo8 = EngineOptions::kPrefillLo8Default;
    o->quant_decode = 1;
    const EngineOptions d;
    o->sparse_window = d.sparse_window;
    o->sparse_global = d.sparse_global;
    o->sparse_threshold = d.sparse_threshold;
}

static EngineOptions to_options(const vsl_engine_options* o) {
    EngineOptions e;
    if (!o) return e;
    e.device = o->device;
    e.kv_capacity = o->kv_capacity;
    e.use_graph = o->use_graph != 0;
    e.prefill_chunk = o->prefill_chunk ? o->prefill_chunk : 2048;
    e.attn_splits = o->attn_splits;
    e.batched_prefill = o->batched_prefill != 0;
    e.prefill_split = o->prefill_split & EngineOptions::kPrefillSplitAll;
    e.prefill_lo8 = o->prefill_lo8 & EngineOptions::kPrefillLo8Stages;
    e.dequant_f32 = o->dequant_f32 != 0;
    e.quant_decode = o->quant_decode != 0;
    e.sparse_attention = o->sparse_attention != 0;
    e.sparse_window = o->sparse_window;
    e.sparse_global = o->sparse_global;
    e.sparse_threshold = o->sparse_threshold;
    return e;
}

static ModelConfig to_config(const vsl_model_spec* s) {
    ModelConfig c;
    c.hidden_size = s->hidden_size;
    c.num_layers = s->num_layers;
    c.num_attention_heads = s->num_heads;
    c.num_key_value_heads = s->num_kv_heads;
    c.intermediate_size = s->intermediate_size;
    c.vocab_size = s->vocab_size;
    c.max_position_embeddings = s->max_position_embeddings;
    c.rope_theta = s->rope_theta;
    c.rms_epsilon = s->rms_eps;
    c.head_dim = s->num_heads ? s->hidden_size / s->num_heads : 0;
    c.use_fp16 = s->dtype == VSL_DT_F16;
    return c;
}

extern "C" int vsl_engine_open(const char* gguf_path, const vsl_engine_options* opt, vsl_engine** out) {
    if (!gguf_path || !out) return fail(VSL_E_INVALID, "vsl_engine_open: null argument");
    *out = nullptr;
    try {
        auto e = std::make_unique<vsl_engine>();
        e->impl = std::make_unique<VulkanSymbioteEngine>(Path(gguf_path), to_options(opt));
        *out = e.release();
        return VSL_OK;
    } catch (const std::exception& ex) {
        return fail(VSL_E_INVALID, ex.what());
    }
}

extern "C" int vsl_engine_open_synthetic(const vsl_model_spec* spec, uint64_t seed, const vsl_engine_options* opt,
                                         vsl_engine** out) {
    if (!spec || !out) return fail(VSL_E_INVALID, "vsl_engine_open_synthetic: null argument");
    *out = nullptr;
    try {
        if (spec->dtype > VSL_WF_Q8_0)
            return fail(VSL_E_UNSUPPORTED, "vsl_engine_open_synthetic: weights are F32, F16, Q4_0, Q4_1 or Q8_0");
        SyntheticSpec s;
        s.config = to_config(spec);
        // quantized: fp16 draws quantized on the device into the decode packs; the expanded packs hold
        // the quantized values in fp16, or exactly in fp32 with dequant_f32
        s.quant_format = spec->dtype >= VSL_WF_Q4_0 ? static_cast<int>(spec->dtype) : -1;
        s.fp16 = spec->dtype == VSL_DT_F16 || (s.quant_format >= 0 && !(opt && opt->dequant_f32));
        s.init_std = spec->init_std > 0 ? spec->init_std : 0.02f;
        s.seed = seed;
        auto e = std::make_unique<vsl_engine>();
        e->impl = std::make_unique<VulkanSymbioteEngine>(s, to_options(opt));
        *out = e.release();
        return VSL_OK;
    } catch (const std::exception& ex) {
        return fail(VSL_E_INVALID, ex.what());
    }
}

extern "C" int vsl_engine_close(vsl_engine* e) {
    delete e;
    return VSL_OK;
}

extern "C" int vsl_engine_generate_ids(vsl_engine* e, const uint32_t* prompt, uint32_t n_prompt, uint32_t max_new,
                                       const vsl_gen_params* params, uint32_t* out_tokens, float* out_logits,
                                       uint32_t* n_out) {
    if (!e || !prompt || !params || (!out_tokens && max_new)) return fail(VSL_E_INVALID, "vsl_engine_generate_ids: null argument");
    try {
        SamplingParams p;
        p.mode = params->mode;
        p.temperature = params->temperature;
        p.top_k = params->top_k;
        p.seed = params->seed;
        p.stop_on_eos = params->stop_on_eos != 0;
        std::vector<uint32_t> ids(prompt, prompt + n_prompt), out;
        std::vector<float> logits;
        int rc = e->impl->generate_ids(ids, max_new, p, out, out_logits ? &logits : nullptr);
        if (rc < 0) {
            const char* why = rc == kErrCapacity ? "prompt + max_new exceeds the KV capacity"
                              : rc == kErrInvalid ? "empty prompt or bad sampling mode"
                              : rc == VSL_E_UNSUPPORTED ? "seeded top-k needs 1 <= min(top_k, vocab) <= VSL_MAX_TOP_K"
                                                        : "generation failed";
            return fail(rc, std::string("vsl_engine_generate_ids: ") + why);
        }
        if (!out.empty()) std::memcpy(out_tokens, out.data(), out.size() * 4);
        if (out_logits && !logits.empty()) std::memcpy(out_logits, logits.data(), logits.size() * 4);
        if (n_out) *n_out = static_cast<uint32_t>(out.size());
        return VSL_OK;
    } catch (const std::exception& ex) {
        return fail(VSL_E_HIP, ex.what());
    }
}

extern "C" int vsl_engine_generate_forced(vsl_engine* e, const uint32_t* prompt, uint32_t n_prompt,
                                          const uint32_t* forced, uint32_t n_forced, uint32_t max_new,
                                          const vsl_gen_params* params, uint32_t* out_tokens, float* out_logits,
                                          uint32_t* n_out) {
    if (!e || !prompt || !params || (!out_tokens && max_new) || (!forced && n_forced))
        return fail(VSL_E_INVALID, "vsl_engine_generate_forced: null argument");
    if (max_new && n_forced + 1 < max_new)
        return fail(VSL_E_INVALID, "vsl_engine_generate_forced: needs max_new - 1 forced ids");
    try {
        SamplingParams p;
        p.mode = params->mode;
        p.temperature = params->temperature;
        p.top_k = params->top_k;
        p.seed = params->seed;
        std::vector<uint32_t> ids(prompt, prompt + n_prompt), hist(forced, forced + n_forced), out;
        std::vector<float> logits;
        int rc = e->impl->generate_ids(ids, max_new, p, out, out_logits ? &logits : nullptr, &hist);
        if (rc < 0) return fail(rc, "vsl_engine_generate_forced: generation failed (capacity, prompt or sampler)");
        if (!out.empty()) std::memcpy(out_tokens, out.data(), out.size() * 4);
        if (out_logits && !logits.empty()) std::memcpy(out_logits, logits.data(), logits.size() * 4);
        if (n_out) *n_out = static_cast<uint32_t>(out.size());
        return VSL_OK;
    } catch (const std::exception& ex) {
        return fail(VSL_E_HIP, ex.what());
    }
}

static SamplingParams to_params(const vsl_gen_params* params) {
    SamplingParams p;
    p.mode = params->mode;
    p.temperature = params->temperature;
    p.top_k = params->top_k;
    p.seed = params->seed;
    p.stop_on_eos = params->stop_on_eos != 0;
    return p;
}

extern "C" int vsl_engine_begin(vsl_engine* e, const uint32_t* prompt, uint32_t n_prompt, uint32_t max_new,
                                const vsl_gen_params* params) {
    if (!e || !prompt || !params) return fail(VSL_E_INVALID, "vsl_engine_begin: null argument");
    try {
        std::vector<uint32_t> ids(prompt, prompt + n_prompt);
        int rc = e->impl->begin_generation(ids, max_new, to_params(params));
        if (rc < 0) return fail(rc, "vsl_engine_begin: empty prompt, max_new == 0, bad mode or KV capacity exceeded");
        return VSL_OK;
    } catch (const std::exception& ex) {
        return fail(VSL_E_HIP, ex.what());
    }
}

extern "C" int vsl_engine_decode(vsl_engine* e, uint32_t n, uint32_t* issued) {
    if (!e) return fail(VSL_E_INVALID, "vsl_engine_decode: null engine");
    try {
        int rc = e->impl->decode_steps(n);
        if (rc < 0) return fail(rc, "vsl_engine_decode: no generation in flight");
        if (issued) *issued = static_cast<uint32_t>(rc);
        return VSL_OK;
    } catch (const std::exception& ex) {
        return fail(VSL_E_HIP, ex.what());
    }
}

extern "C" int vsl_engine_sync(vsl_engine* e) {
    if (!e) return fail(VSL_E_INVALID, "vsl_engine_sync: null engine");
    try {
        e->impl->synchronize();
        return VSL_OK;
    } catch (const std::exception& ex) {
        return fail(VSL_E_HIP, ex.what());
    }
}

extern "C" int vsl_engine_finish(vsl_engine* e, uint32_t* out_tokens, uint32_t* n_out) {
    if (!e || !out_tokens) return fail(VSL_E_INVALID, "vsl_engine_finish: null argument");
    try {
        std::vector<uint32_t> out;
        int rc = e->impl->finish_generation(out);
        if (rc < 0) return fail(rc, "vsl_engine_finish: no generation in flight or KV capacity exceeded");
        if (!out.empty()) std::memcpy(out_tokens, out.data(), out.size() * 4);
        if (n_out) *n_out = static_cast<uint32_t>(out.size());
        return VSL_OK;
    } catch (const std::exception& ex) {
        return fail(VSL_E_HIP, ex.what());
    }
}

extern "C" int vsl_engine_time_op(vsl_engine* e, int op, uint32_t iterations, double* avg_ms) {
    if (!e || !avg_ms || op < 0 || op > 5 || iterations == 0) return fail(VSL_E_INVALID, "vsl_engine_time_op: bad argument");
    try {
        *avg_ms = e->impl->time_op(op, iterations);
        return VSL_OK;
    } catch (const std::exception& ex) {
        return fail(VSL_E_HIP, ex.what());
    }
}

extern "C" int vsl_engine_generate_text(vsl_engine* e, const char* prompt, uint32_t max_tokens, float temperature,
                                        char* out, uint64_t out_cap, uint64_t* out_len) {
    if (!e || !prompt) return fail(VSL_E_INVALID, "vsl_engine_generate_text: null argument");
    try {
        std::string r = e->impl->generate(prompt, max_tokens, temperature);
        if (out_len) *out_len = r.size();
        if (out && out_cap) {
            size_t n = r.size() < out_cap - 1 ? r.size() : out_cap - 1;
            std::memcpy(out, r.data(), n);
            out[n] = 0;
        }
        return VSL_OK;
    } catch (const std::exception& ex) {
        return fail(VSL_E_HIP, ex.what());
    }
}

extern "C" int vsl_engine_get_config(vsl_engine* e, vsl_model_spec* s) {
    if (!e || !s) return fail(VSL_E_INVALID, "vsl_engine_get_config: null argument");
    const ModelConfig& c = e->impl->config();
    s->hidden_size = c.hidden_size;
    s->num_layers = c.num_layers;
    s->num_heads = c.num_attention_heads;
    s->num_kv_heads = c.num_key_value_heads;
    s->intermediate_size = c.intermediate_size;
    s->vocab_size = c.vocab_size;
    s->max_position_embeddings = c.max_position_embeddings;
    s->rope_theta = c.rope_theta;
    s->rms_eps = c.rms_epsilon;
    s->init_std = 0.0f;
    s->dtype = e->impl->weights_fp16() ? VSL_DT_F16 : VSL_DT_F32;
    s->head_dim = c.head_dim;
    return VSL_OK;
}

extern "C" int vsl_engine_last_stats(vsl_engine* e, vsl_gen_stats* s) {
    if (!e || !s) return fail(VSL_E_INVALID, "vsl_engine_last_stats: null argument");
    const GenerationTimings& t = e->impl->last_timings();
    s->prompt_tokens = t.prompt_tokens;
    s->generated_tokens = t.generated_tokens;
    s->kv_positions = t.kv_positions;
    s->pad = 0;
    s->prefill_ms = t.prefill_ms;
    s->decode_ms = t.decode_ms;
    return VSL_OK;
}

extern "C" int vsl_engine_vram_stats(vsl_engine* e, vsl_pool_stats* s) {
    if (!e || !s) return fail(VSL_E_INVALID, "vsl_engine_vram_stats: null argument");
    MemoryPoolStats m = e->impl->get_vram_stats();
    s->total_size = m.total_size;
    s->used_size = m.used_size;
    s->free_size = m.free_size;
    s->allocation_count = m.allocation_count;
    s->fragmentation_ratio = m.fragmentation_ratio;
    return VSL_OK;
}

extern "C" int vsl_engine_kv_bytes(vsl_engine* e, uint64_t* out) {
    if (!e || !out) return fail(VSL_E_INVALID, "vsl_engine_kv_bytes: null argument");
    *out = e->impl->get_kv_cache_memory_usage();
    return VSL_OK;
}

extern "C" int vsl_engine_weight_bytes(vsl_engine* e, uint64_t* out) {
    if (!e || !out) return fail(VSL_E_INVALID, "vsl_engine_weight_bytes: null argument");
    *out = e->impl->weight_bytes();
    return VSL_OK;
}

extern "C" int vsl_engine_clear_kv(vsl_engine* e) {
    if (!e) return fail(VSL_E_INVALID, "vsl_engine_clear_kv: null engine");
    e->impl->clear_kv_cache();
    return VSL_OK;
}

extern "C" int vsl_engine_benchmark(vsl_engine* e, uint32_t warmup, uint32_t tokens, uint32_t iterations, double* avg_tps,
                                    double* min_tps, double* max_tps) {
    if (!e) return fail(VSL_E_INVALID, "vsl_engine_benchmark: null engine");
    try {
        BenchmarkResult r = e->impl->run_benchmark(warmup, tokens, iterations);
        if (avg_tps) *avg_tps = r.avg_tokens_per_sec;
        if (min_tps) *min_tps = r.min_tokens_per_sec;
        if (max_tps) *max_tps = r.max_tokens_per_sec;
        return VSL_OK;
    } catch (const std::exception& ex) {
        return fail(VSL_E_HIP, ex.what());
    }
}

extern "C" int vsl_engine_read_tensor(vsl_engine* e, const char* name, void* dst, uint64_t bytes, int* dtype_out) {
    if (!e || !name || !dst) return fail(VSL_E_INVALID, "vsl_engine_read_tensor: null argument");
    auto r = e->impl->read_tensor(name, dst, bytes, dtype_out);
    if (!r.has_value()) return fail(r.error(), std::string("vsl_engine_read_tensor: cannot read ") + name);
    return VSL_OK;
}

extern "C" int vsl_write_synthetic_gguf(const char* path, const vsl_model_spec* spec, uint64_t seed, int convention) {
    if (!path || !spec) return fail(VSL_E_INVALID, "vsl_write_synthetic_gguf: null argument");
    if (spec->dtype > VSL_WF_Q8_0) return fail(VSL_E_INVALID, "vsl_write_synthetic_gguf: unknown weight format");
    SyntheticSpec s;
    s.config = to_config(spec);
    s.fp16 = spec->dtype == VSL_DT_F16;
    s.quant_format = spec->dtype >= VSL_WF_Q4_0 ? static_cast<int>(spec->dtype) : -1;
    s.init_std = spec->init_std > 0 ? spec->init_std : 0.02f;
    s.seed = seed;
    auto r = write_synthetic_gguf(Path(path), s, convention == 1 ? GGUFConvention::GGML : GGUFConvention::REFERENCE);
    if (!r.has_value()) return fail(r.error(), "vsl_write_synthetic_gguf: write failed");
    return VSL_OK;
}

extern "C" int vsl_write_synthetic_gguf_vocab(const char* path, const vsl_model_spec* spec, uint64_t seed,
                                              int convention, const char* const* tokens, const uint64_t* token_lens,
                                              uint32_t n_tokens, int keyed) {
    if (!path || !spec || (n_tokens && (!tokens || !token_lens)))
        return fail(VSL_E_INVALID, "vsl_write_synthetic_gguf_vocab: null argument");
    if (spec->dtype > VSL_WF_Q8_0) return fail(VSL_E_INVALID, "vsl_write_synthetic_gguf_vocab: unknown weight format");
    SyntheticSpec s;
    s.config = to_config(spec);
    s.fp16 = spec->dtype == VSL_DT_F16;
    s.quant_format = spec->dtype >= VSL_WF_Q4_0 ? static_cast<int>(spec->dtype) : -1;
    s.init_std = spec->init_std > 0 ? spec->init_std : 0.02f;
    s.seed = seed;
    for (uint32_t i = 0; i < n_tokens; ++i) {
        if (!tokens[i] && token_lens[i]) return fail(VSL_E_INVALID, "vsl_write_synthetic_gguf_vocab: null token");
        s.vocab.emplace_back(tokens[i] ? tokens[i] : "", static_cast<size_t>(token_lens[i]));
    }
    s.vocab_keyed = keyed != 0;
    auto r = write_synthetic_gguf(Path(path), s, convention == 1 ? GGUFConvention::GGML : GGUFConvention::REFERENCE);
    if (!r.has_value()) return fail(r.error(), "vsl_write_synthetic_gguf_vocab: write failed");
    return VSL_OK;
}

// Packs
static void fill_pack(const PackMetadata& m, vsl_pack_info* o, char* name, uint64_t cap) {
    std::memset(o, 0, sizeof(*o));
    o->pack_id = m.pack_id;
    o->type = static_cast<int32_t>(m.type);
    o->layer_idx = m.layer_idx;
    o->head_idx = m.head_idx;
    o->alignment = m.alignment;
    o->compressed_size = m.compressed_size;
    o->decompressed_size = m.decompressed_size;
    o->file_offset = m.file_offset;
    o->base_priority = m.base_priority;
    o->tier = -1;
    o->dtype = -1;
    o->n_dimensions = m.n_dimensions;
    if (name && cap) {
        const size_t n = std::min<size_t>(m.tensor_name.size(), static_cast<size_t>(cap - 1));
        std::memcpy(name, m.tensor_name.data(), n);
        name[n] = 0;
    }
}

extern "C" int vsl_engine_pack_count(vsl_engine* e, uint64_t* n) {
    if (!e || !n) return fail(VSL_E_INVALID, "vsl_engine_pack_count: null argument");
    *n = e->impl->packs().size();
    return VSL_OK;
}

extern "C" int vsl_engine_pack(vsl_engine* e, uint64_t idx, vsl_pack_info* out, char* name, uint64_t name_cap) {
    if (!e || !out) return fail(VSL_E_INVALID, "vsl_engine_pack: null argument");
    const auto& packs = e->impl->packs();
    if (idx >= packs.size()) return fail(kErrNotFound, "vsl_engine_pack: index out of range");
    const ResidentPack& p = packs[idx];
    fill_pack(p.meta, out, name, name_cap);
    out->tier = static_cast<int32_t>(p.tier);
    out->dtype = p.dtype;
    out->resident_bytes = p.bytes;
    out->device_ptr = p.device_ptr;
    return VSL_OK;
}

// Tokenizer
struct vsl_tokenizer {
    std::unique_ptr<Tokenizer> impl;
};

extern "C" int vsl_tokenizer_open(const char* gguf_path, vsl_tokenizer** out) {
    if (!out) return fail(VSL_E_INVALID, "vsl_tokenizer_open: null argument");
    auto t = std::make_unique<vsl_tokenizer>();
    t->impl = gguf_path ? Tokenizer::from_gguf(Path(gguf_path)) : Tokenizer::create_simple_tokenizer();
    *out = t.release();
    return VSL_OK;
}

extern "C" int vsl_tokenizer_close(vsl_tokenizer* t) {
    delete t;
    return VSL_OK;
}

extern "C" int vsl_tokenizer_info(vsl_tokenizer* t, uint32_t* vocab_size, int* source) {
    if (!t) return fail(VSL_E_INVALID, "vsl_tokenizer_info: null handle");
    if (vocab_size) *vocab_size = t->impl->vocab_size();
    if (source) *source = static_cast<int>(t->impl->source());
    return VSL_OK;
}

extern "C" int vsl_tokenizer_encode(vsl_tokenizer* t, const char* text, uint64_t text_len, uint32_t* ids, uint64_t cap,
                                    uint64_t* n_out) {
    if (!t || (!text && text_len) || (!ids && cap) || !n_out) return fail(VSL_E_INVALID, "vsl_tokenizer_encode: null argument");
    const std::vector<uint32_t> r = t->impl->encode(std::string(text ? text : "", static_cast<size_t>(text_len)));
    for (uint64_t i = 0; i < r.size() && i < cap; ++i) ids[i] = r[i];
    *n_out = r.size();
    return VSL_OK;
}

extern "C" int vsl_tokenizer_decode(vsl_tokenizer* t, const uint32_t* ids, uint64_t n, char* out, uint64_t cap,
                                    uint64_t* len_out) {
    if (!t || (!ids && n) || (!out && cap) || !len_out) return fail(VSL_E_INVALID, "vsl_tokenizer_decode: null argument");
    const std::string r = t->impl->decode(std::vector<uint32_t>(ids, ids + n));
    if (cap) std::memcpy(out, r.data(), static_cast<size_t>(std::min<uint64_t>(cap, r.size())));
    *len_out = r.size();
    return VSL_OK;
}

extern "C" int vsl_synthetic_fill_host(void* out, int dtype, uint64_t n, uint64_t seed, const char* name, float mean,
                                       float stddev) {
    if (!out || !name) return fail(VSL_E_INVALID, "vsl_synthetic_fill_host: null argument");
    synthetic_fill_host(out, dtype == VSL_DT_F16, n, seed, name, mean, stddev);
    return VSL_OK;
}

extern "C" int vsl_config_load_args(int argc, const char* const* argv) {
    std::vector<char*> v;
    v.reserve(argc + 1);
    for (int i = 0; i < argc; ++i) v.push_back(const_cast<char*>(argv[i]));
    v.push_back(nullptr);
    try {
        ConfigManager::instance().load_from_args(argc, v.data());
    } catch (const std::exception& ex) {
        return fail(VSL_E_INVALID, ex.what());
    }
    return VSL_OK;
}

extern "C" int vsl_config_load_file(const char* path) {
    if (!path) return fail(VSL_E_INVALID, "vsl_config_load_file: null path");
    return ConfigManager::instance().load_from_file(Path(path)) ? VSL_OK : fail(VSL_E_INVALID, "config file invalid");
}

extern "C" int vsl_config_save_file(const char* path) {
    if (!path) return fail(VSL_E_INVALID, "vsl_config_save_file: null path");
    return ConfigManager::instance().save_to_file(Path(path)) ? VSL_OK : fail(VSL_E_INVALID, "cannot write config");
}

extern "C" int vsl_config_reset(void) {
    ConfigManager::instance().set_defaults();
    return VSL_OK;
}

extern "C" int vsl_config_get(int* enable_gpu, int* device, uint32_t* kv_capacity, uint64_t* seed, float* vram_budget_gb) {
    const ConfigManager& c = ConfigManager::instance();
    if (enable_gpu) *enable_gpu = c.performance().enable_gpu ? 1 : 0;
    if (device) *device = c.performance().device;
    if (kv_capacity) *kv_capacity = c.performance().kv_capacity;
    if (seed) *seed = c.performance().seed;
    if (vram_budget_gb) *vram_budget_gb = c.memory().vram_budget_gb;
    return VSL_OK;
}

// ------------------------------------------------------------------------------------------
// GGUFLoader
// ------------------------------------------------------------------------------------------
struct vsl_gguf {
    std::unique_ptr<GGUFLoader> impl;
};

extern "C" int vsl_gguf_open(const char* path, vsl_gguf** out) {
    if (!path || !out) return fail(VSL_E_INVALID, "vsl_gguf_open: null argument");
    *out = nullptr;
    auto g = std::make_unique<vsl_gguf>();
    g->impl = std::make_unique<GGUFLoader>(Path(path));
    auto r = g->impl->load();
    if (!r.has_value()) return fail(r.error(), std::string("vsl_gguf_open: cannot parse ") + path);
    *out = g.release();
    return VSL_OK;
}

extern "C" int vsl_gguf_pack_count(vsl_gguf* g, uint64_t* n) {
    if (!g || !n) return fail(VSL_E_INVALID, "vsl_gguf_pack_count: null argument");
    *n = g->impl->tensor_count();
    return VSL_OK;
}

extern "C" int vsl_gguf_pack(vsl_gguf* g, uint64_t idx, vsl_pack_info* out, char* name, uint64_t name_cap) {
    if (!g || !out) return fail(VSL_E_INVALID, "vsl_gguf_pack: null argument");
    const std::vector<PackMetadata> packs = g->impl->generate_packs(g->impl->get_model_config());
    if (idx >= packs.size()) return fail(kErrNotFound, "vsl_gguf_pack: index out of range");
    fill_pack(packs[idx], out, name, name_cap);
    return VSL_OK;
}

extern "C" int vsl_gguf_close(vsl_gguf* g) {
    delete g;
    return VSL_OK;
}

extern "C" int vsl_gguf_info(vsl_gguf* g, uint64_t* tensor_count, uint64_t* metadata_count, uint32_t* version,
                             int* convention, uint64_t* data_start) {
    if (!g) return fail(VSL_E_INVALID, "vsl_gguf_info: null handle");
    if (tensor_count) *tensor_count = g->impl->tensor_count();
    if (metadata_count) *metadata_count = g->impl->metadata_count();
    if (version) *version = g->impl->get_version();
    if (convention) *convention = static_cast<int>(g->impl->convention());
    if (data_start) *data_start = g->impl->data_start();
    return VSL_OK;
}

extern "C" int vsl_gguf_model_config(vsl_gguf* g, vsl_model_spec* s) {
    if (!g || !s) return fail(VSL_E_INVALID, "vsl_gguf_model_config: null argument");
    ModelConfig c = g->impl->get_model_config();
    s->hidden_size = c.hidden_size;
    s->num_layers = c.num_layers;
    s->num_heads = c.num_attention_heads;
    s->num_kv_heads = c.num_key_value_heads;
    s->intermediate_size = c.intermediate_size;
    s->vocab_size = c.vocab_size;
    s->max_position_embeddings = c.max_position_embeddings;
    s->rope_theta = c.rope_theta;
    s->rms_eps = c.rms_epsilon;
    s->init_std = 0.0f;
    s->dtype = c.use_fp16 ? VSL_DT_F16 : VSL_DT_F32;
    s->head_dim = c.head_dim;
    return VSL_OK;
}

extern "C" int vsl_gguf_tensor(vsl_gguf* g, const char* name, uint64_t* data_offset, uint64_t* data_size,
                               uint32_t* raw_type, uint32_t* n_dims, uint64_t dims[4]) {
    if (!g || !name) return fail(VSL_E_INVALID, "vsl_gguf_tensor: null argument");
    const GGUFTensorInfo* t = g->impl->get_tensor(name);
    if (!t) return fail(kErrNotFound, std::string("vsl_gguf_tensor: no tensor ") + name);
    if (data_offset) *data_offset = t->data_offset;
    if (data_size) *data_size = t->data_size;
    if (raw_type) *raw_type = static_cast<uint32_t>(t->data_type);
    if (n_dims) *n_dims = t->n_dimensions;
    if (dims)
        for (int i = 0; i < 4; ++i) dims[i] = i < (int)t->dimensions.size() ? t->dimensions[i] : 1;
    return VSL_OK;
}

extern "C" int64_t vsl_gguf_read_f32(vsl_gguf* g, const char* name, float* out, uint64_t cap) {
    if (!g || !name || !out) return fail(VSL_E_INVALID, "vsl_gguf_read_f32: null argument");
    const GGUFTensorInfo* t = g->impl->get_tensor(name);
    if (!t) return fail(kErrNotFound, std::string("vsl_gguf_read_f32: no tensor ") + name);
    auto r = g->impl->read_tensor_data(*t, true);
    if (!r.has_value()) return fail(r.error(), std::string("vsl_gguf_read_f32: cannot read ") + name);
    const auto& v = r.value();
    if (v.size() > cap) return fail(kErrCapacity, "vsl_gguf_read_f32: output too small");
    std::memcpy(out, v.data(), v.size() * 4);
    return static_cast<int64_t>(v.size());
}
