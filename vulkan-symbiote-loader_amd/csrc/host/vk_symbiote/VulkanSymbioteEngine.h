// VulkanSymbioteEngine.h -- the reference's engine API (vk_symbiote/include/vk_symbiote/
// VulkanSymbioteEngine.h:72-118) on an MI355X HIP backend.
//
// Kept: the path constructor, generate / encode / decode, config(), run_benchmark(_detailed),
// generate_text_batch, get_vram_stats / get_peak_vram_usage, clear_kv_cache /
// get_kv_cache_memory_usage, get_performance_metrics / reset_performance_metrics.
// Dropped (Vulkan-typed): the GUI constructor taking Vk handles and device() /
// physical_device() / compute_queue().
// Added: a token-id entry point (generate_ids) with explicit sampling parameters and optional
// logits, engine options, a synthetic-weights constructor, per-generation timings, and
// read_tensor (device -> host copy of one pack).
#pragma once

#include <map>
#include <array>
#include <memory>
#include <string>
#include <tuple>
#include <unordered_map>
#include <vector>

#include "Common.h"
#include "GGUFLoader.h"
#include "NomadPack.h"
#include "Tokenizer.h"

struct vsl_arena;
struct vsl_graph;
struct vsl_ctrl;

namespace vk_symbiote {

struct BenchmarkResult {
    uint32_t warmup_tokens = 0;
    uint32_t benchmark_tokens = 0;
    uint32_t iterations = 0;
    double avg_tokens_per_sec = 0.0;
    double min_tokens_per_sec = 0.0;
    double max_tokens_per_sec = 0.0;
    double std_dev_tokens_per_sec = 0.0;
    double avg_latency_ms = 0.0;
    double peak_vram_gb = 0.0;
    double cache_hit_rate = 0.0;
    double cache_size_mb = 0.0;
    std::unordered_map<std::string, double> power_mode_results;
    double memory_pressure_result = 0.0;
};

struct BenchmarkStats {
    double avg_tokens_per_sec = 0.0;
    double min_tokens_per_sec = 0.0;
    double max_tokens_per_sec = 0.0;
    double std_dev_tokens_per_sec = 0.0;
    double avg_latency_ms = 0.0;
    double peak_vram_gb = 0.0;
    double avg_vram_usage_gb = 0.0;
    double fragmentation_ratio = 0.0;
    double cache_hit_rate = 0.0;
    uint64_t total_evictions = 0;
    double eviction_rate = 0.0;
    void print() const;
};

struct EngineOptions {
    int device = 0;
    uint32_t kv_capacity = 0;     // 0 = min(max_position_embeddings, 4096)
    bool use_graph = true;        // capture each decode step once, replay it
    uint32_t prefill_chunk = 2048;
    uint32_t attn_splits = 0;     // 0 = 32 splits
    bool batched_prefill = true;  // fp16 models: MFMA prefill (else token by token)
    // Which prefill activations are carried as hi/lo fp16 pairs (two MFMAs per tile, ~22-bit
    // inputs) instead of one rounded fp16 value: bit 0 QKV GEMM input, bit 1 attention (q and the
    // probabilities), bit 2 O-projection input, bit 3 gate/up GEMM input, bit 4 down-projection input.
    uint32_t prefill_split = kPrefillSplitAll;
    // Which of the split stages carry their lo part as fp8 e4m3 (VSL_DT_F16F8: ~15-bit inputs, the
    // lo plane multiplied on the fp8 matrix cores) instead of a second fp16 plane: bit 0 QKV input,
    // bit 2 O-projection input (the attention output), bit 3 gate/up input, bit 4 down input (the
    // attention's own q / probabilities have no fp8 form).
    // Taken where the shapes allow it (model width and FFN size multiples of 256, the QKV width a
    // multiple of 256) and, per prompt chunk, where the stage's GEMMs run on the direct-to-LDS tiles
    // at full occupancy (vsl_gemm_f16_direct; e.g. not the 1B model's 128-row gate/up, where the fp8
    // form would force 64 tiles: 1.96 -> 2.24 ms); elsewhere the stage keeps the fp16 lo plane. The
    // default takes the O, gate/up and down inputs: on the 8B model their fp8 form leaves the logit
    // error against fp32 inputs about level (0.0026 against 0.0023 max-abs), while an fp8 QKV input
    // doubles it (0.0052; the attention scores amplify it) for 0.15 ms of a 13 ms 512-token prompt.
    uint32_t prefill_lo8 = kPrefillLo8Default;
    // Block-quantized GGUF weights (Q4_0 / Q4_1 / Q8_0) are expanded at load into fp16 packs, or into
    // fp32 packs holding exactly the values the reference's dequantize_tensor returns when set.
    bool dequant_f32 = false;
    // Block-quantized weights also stay resident as blocks (vsl_quant_pack: 9 / 5 / 6 bits per weight
    // for Q8_0 / Q4_0 / Q4_1) and the decode GEMVs multiply those directly, reading 31 to 56 % of the
    // fp16 bytes per token; the prompt pass keeps its MFMA GEMMs on the expanded packs. Taken per
    // operand ([Wq; Wk; Wv], Wo, [Wgate; Wup], Wdown, the output projection) when its tensors share
    // one quantized format and its input width is a multiple of 32.
    bool quant_decode = true;
    // Windowed long-context mode (the reference's use_sparse_attention, Common.h:70-75, taken when
    // seq_len > 8192, VulkanSymbioteEngine.cpp:788): a query at position p with p + 1 > threshold
    // attends to the first sparse_global keys and to the sparse_window keys before it (and itself)
    // only.  Off by default: every length then runs exact dense causal attention.
    bool sparse_attention = false;
    uint32_t sparse_window = 512;
    uint32_t sparse_global = 16;
    uint32_t sparse_threshold = 8192;
    bool verbose = false;
    static constexpr uint32_t kPrefillSplitAll = 0x1F;
    static constexpr uint32_t kPrefillLo8Stages = 0x1D;
    static constexpr uint32_t kPrefillLo8Default = 0x1C;
};

// Synthetic Llama-style model: every linear weight ~ N(0, init_std) from the Philox stream keyed by
// (seed, tensor name), norm gains 1.0.
struct SyntheticSpec {
    ModelConfig config;
    bool fp16 = true;
    // VSL_WF_Q4_0 / Q4_1 / Q8_0: write_synthetic_gguf stores every 2-D weight (embeddings and output
    // included) block-quantized from the fp32 draws; a synthetic engine draws fp16 weights, quantizes
    // every linear weight on the device (vsl_quantize_pack) into the decode packs and replaces the
    // fp16 packs with the quantized values (the embedding stays fp16). -1 keeps F16 / F32 per `fp16`.
    int quant_format = -1;
    // write_synthetic_gguf only: a vocabulary, written as the string array "tokenizer.ggml.tokens"
    // or, with vocab_keyed, as one string key "tokenizer.ggml.tokens.<id>" per entry
    std::vector<std::string> vocab;
    bool vocab_keyed = false;
    float init_std = 0.02f;
    uint64_t seed = 0;
};

struct SamplingParams {
    int mode = 0;  // VSL_SAMPLE_*
    float temperature = 0.0f;
    uint32_t top_k = 40;
    uint64_t seed = 0;
    bool stop_on_eos = true;
};

struct GenerationTimings {
    uint32_t prompt_tokens = 0;
    uint32_t generated_tokens = 0;
    double prefill_ms = 0.0;  // prompt processing up to and including the first sampled token
    double decode_ms = 0.0;   // the remaining generated_tokens - 1 decode steps
    uint32_t kv_positions = 0;
};

class VulkanSymbioteEngine {
   public:
    explicit VulkanSymbioteEngine(const Path& model_path);
    VulkanSymbioteEngine(const Path& model_path, const EngineOptions& options);
    VulkanSymbioteEngine(const SyntheticSpec& spec, const EngineOptions& options);
    ~VulkanSymbioteEngine();
    VulkanSymbioteEngine(const VulkanSymbioteEngine&) = delete;
    VulkanSymbioteEngine& operator=(const VulkanSymbioteEngine&) = delete;

    std::string generate(const std::string& prompt, uint32_t max_tokens = 256, float temperature = 0.7f);
    std::vector<uint32_t> encode(const std::string& text);
    std::string decode(const std::vector<uint32_t>& tokens);
    const Tokenizer& tokenizer() const { return *tokenizer_; }

    // Token-id entry point.  Returns the number of generated tokens (<0 on error).
    // logits_out (optional) receives one vocab-sized row per generated token: the logits that
    // token was sampled from.  forced (optional, >= max_new - 1 ids) teacher-forces the history:
    // step t + 1 takes forced[t] as its input instead of the token sampled at step t (the sampled
    // tokens are still returned, and EOS does not stop the run), so every step's logits can be
    // compared with another implementation's on the same token history.
    int generate_ids(const std::vector<uint32_t>& prompt, uint32_t max_new, const SamplingParams& params,
                     std::vector<uint32_t>& out_tokens, std::vector<float>* logits_out = nullptr,
                     const std::vector<uint32_t>* forced = nullptr);

    const ModelConfig& config() const noexcept { return config_; }
    ModelConfig& config() noexcept { return config_; }

    BenchmarkResult run_benchmark(uint32_t warmup_tokens = 10, uint32_t benchmark_tokens = 100, uint32_t iterations = 3);
    BenchmarkStats run_benchmark_detailed(uint32_t warmup_tokens, uint32_t benchmark_tokens, uint32_t iterations);
    std::vector<std::string> generate_text_batch(const std::vector<std::string>& prompts,
                                                 uint32_t max_tokens_per_prompt = 256, float temperature = 0.7f);

    MemoryPoolStats get_vram_stats();
    double get_peak_vram_usage();
    void clear_kv_cache();
    size_t get_kv_cache_memory_usage() const;

    const PerformanceMetrics& get_performance_metrics() const { return performance_metrics_; }
    void reset_performance_metrics() { performance_metrics_.reset(); }

    // Split form of generate_ids: begin_generation runs the prompt and samples the first token;
    // decode_steps enqueues n decode steps (asynchronous); finish_generation waits and collects.
    int begin_generation(const std::vector<uint32_t>& prompt, uint32_t max_new, const SamplingParams& params);
    int decode_steps(uint32_t n);
    int finish_generation(std::vector<uint32_t>& out_tokens);
    void synchronize();
    // Average duration (ms) of one launch of a decode-step op, timed with HIP events on the engine's
    // stream over `iterations` rounds that visit every layer (so no weight is re-read from cache).
    // op: 0 qkv+rope+kv, 1 attention, 2 o-proj, 3 norm+gate/up+swiglu, 4 down-proj, 5 lm_head+sample.
    double time_op(int op, uint32_t iterations);

    // additive
    const GenerationTimings& last_timings() const { return timings_; }
    const EngineOptions& options() const { return options_; }
    const std::vector<ResidentPack>& packs() const { return pack_manager_.packs(); }
    ExpectedVoid read_tensor(const std::string& name, void* host_dst, size_t bytes, int* dtype_out = nullptr);
    uint32_t kv_capacity() const { return cap_; }
    bool weights_fp16() const { return wdt_ == 1; }
    uint64_t weight_bytes() const { return weight_bytes_; }

   private:
    struct Layer {
        float* attn_norm = nullptr;
        float* ffn_norm = nullptr;
        void* wqkv = nullptr;
        void* wo = nullptr;
        void* wgu = nullptr;
        void* wdown = nullptr;
        void* kc = nullptr;
        void* vc = nullptr;
        // VSL_GEMM_B8_SHIFT flags of the fp8 lo products against [Wq; Wk; Wv], Wo, [Wgate; Wup], Wdown:
        // each matrix's own shift, from its largest weight (measure_weight_ranges)
        int b8_qkv = 0, b8_o = 0, b8_gu = 0, b8_down = 0;
        // resident block-quantized packs of the same operands for the decode GEMVs (nullptr: none)
        // and their VSL_DT_Q* dtypes
        void* qqkv = nullptr;
        void* qo = nullptr;
        void* qgu = nullptr;
        void* qdown = nullptr;
        int qdt_qkv = 0, qdt_o = 0, qdt_gu = 0, qdt_down = 0;
    };
    // VSL_WF_* format of each decode operand's resident pack, -1 for none: per layer [Wq; Wk; Wv],
    // Wo, [Wgate; Wup], Wdown; and the output projection
    std::vector<std::array<int, 4>> qfmt_;
    int qfmt_out_ = -1;
    void plan_quant_gguf(const ModelConfig& cfg);
    void plan_quant_uniform(const ModelConfig& cfg, int fmt);

    ModelConfig config_;
    EngineOptions options_;
    PerformanceMetrics performance_metrics_;
    GenerationTimings timings_;
    PackManager pack_manager_;
    std::unique_ptr<GGUFLoader> loader_;
    std::unique_ptr<Tokenizer> tokenizer_;

    int wdt_ = 1, kvdt_ = 1, edt_ = 1;  // VSL_DT_* of linear weights, KV cache, embedding
    uint32_t cap_ = 0, nsplit_ = 32;
    uint64_t weight_bytes_ = 0, kv_bytes_ = 0;
    double peak_vram_gb_ = 0.0;

    vsl_arena* arena_ = nullptr;
    void* stream_ = nullptr;
    void* upload_stream_ = nullptr;
    void* ev_[4] = {nullptr, nullptr, nullptr, nullptr};

    // device buffers
    void* embed_ = nullptr;
    void* out_w_ = nullptr;
    void* out_q_ = nullptr;  // the output projection's block-quantized pack (nullptr: none)
    int out_qdt_ = 0;
    // the output projection operand of the lm_head GEMV: its pack where it has one
    const void* lm_w() const { return out_q_ ? out_q_ : out_w_; }
    int lm_dt() const { return out_q_ ? out_qdt_ : wdt_; }
    float* out_norm_ = nullptr;
    std::vector<Layer> layers_;
    float* rope_cos_ = nullptr;
    float* rope_sin_ = nullptr;
    float *x_ = nullptr, *q_ = nullptr, *attn_ = nullptr, *h_ = nullptr, *logits_ = nullptr;
    float* wrange_ = nullptr;  // [L][4] largest weight magnitudes (measure_weight_ranges)
    float *part_o_ = nullptr, *part_ml_ = nullptr;
    float* lm_val_ = nullptr;
    uint32_t* lm_idx_ = nullptr;
    uint32_t* tokens_ = nullptr;
    uint32_t* prompt_dev_ = nullptr;
    vsl_ctrl* ctrl_ = nullptr;
    // prefill (fp16 MFMA path)
    uint32_t chunk_ = 0;
    float *px_ = nullptr, *pqkv_ = nullptr;
    void *pxn_ = nullptr, *pq_ = nullptr, *pattn_ = nullptr, *ph_ = nullptr;
    void* gws_ = nullptr;  // split-K workspace of the prefill GEMMs
    uint64_t gws_bytes_ = 0;
    // pinned host mirrors
    uint32_t* host_tokens_ = nullptr;
    vsl_ctrl* host_ctrl_ = nullptr;

    std::map<std::tuple<int, uint32_t, uint32_t, uint64_t>, vsl_graph*> graphs_;
    // state of the generation in flight
    SamplingParams gen_params_;
    uint32_t gen_prompt_ = 0, gen_max_new_ = 0, gen_issued_ = 0;
    bool gen_active_ = false;

    void init_device(const ModelConfig& cfg, bool fp16_weights, int embed_dtype);
    void plan_and_allocate();
    void upload_rope_tables();
    void load_weights_from_gguf();
    void init_synthetic_weights(const SyntheticSpec& spec);
    void enqueue_layers(uint32_t l0, uint32_t l1);
    void enqueue_step(const SamplingParams& p);
    void prefill_tokenwise(uint32_t n_prompt, const SamplingParams& p);
    void prefill_batched(uint32_t n_prompt, const SamplingParams& p);
    // the stages of options_.prefill_lo8 whose GEMM shapes have the fp8 lo form
    uint32_t prefill_lo8_stages() const;
    // the fp8 lo products' weight shifts of every layer (Layer::b8_*), from each fp16 matrix's largest
    // finite magnitude, so that no weight leaves e4m3's range
    void measure_weight_ranges();
    vsl_graph* step_graph(const SamplingParams& p);
    void release();
    void check(int rc, const char* what) const;
    int attend(const Layer& y, float scale);  // decode attention of one layer (dense or windowed)
};

// Writes a synthetic Llama-style GGUF (tensor names as the reference reads them,
// VulkanSymbioteEngine.cpp:2145-2213; linear weights N(0, init_std), norm gains 1.0).
ExpectedVoid write_synthetic_gguf(const Path& path, const SyntheticSpec& spec, GGUFConvention conv);

// Host generator shared by the GGUF writer: Philox4x32-10 keyed by (seed, hash_string(name)),
// Box-Muller in fp64; out is binary16 when fp16 else binary32.
void synthetic_fill_host(void* out, bool fp16, uint64_t n, uint64_t seed, const std::string& name, float mean,
                         float stddev);


}  // namespace vk_symbiote
