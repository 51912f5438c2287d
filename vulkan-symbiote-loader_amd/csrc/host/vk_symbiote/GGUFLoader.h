// GGUFLoader.h -- GGUF reader/writer with the reference's public API
// (vk_symbiote/include/vk_symbiote/GGUFLoader.h:265-333).
//
// Differences from the reference, all on purpose:
//  - the file is memory-mapped and read without a shared stream, so concurrent reads are safe
//    (the reference's read_tensors_parallel shares one std::ifstream across pool threads,
//    GGUFLoader.cpp:761-773 via :1419-1435);
//  - tensor-type ids are read in either convention: the reference's own enum (F32 = 6, F16 = 48,
//    GGUFLoader.h:18-73) with the data section starting right after the tensor infos
//    (GGUFLoader.cpp:653-659), or ggml's (F32 = 0, F16 = 1) with general.alignment padding.
//    The convention is taken from the key "vsl.tensor_type_convention" when present, else
//    inferred from the ids in the file;
//  - F16 tensors are converted by read_tensor_data (the reference routes id 48 into its
//    quantized branch, which rejects it with -20);
//  - Q4_0 / Q4_1 / Q8_0 are dequantized as dequantize_tensor does (GGUFLoader.cpp:1121-1223) in
//    files with the reference's ids, and with ggml's published block layout in files with ggml's
//    ids (which the reference cannot read at all).
#pragma once

#include <chrono>
#include <cstdint>
#include <list>
#include <memory>
#include <mutex>
#include <string>
#include <unordered_map>
#include <vector>

#include "Common.h"
#include "NomadPack.h"

namespace vk_symbiote {

// Every id of the reference's enum (GGUFLoader.h:18-73), so that caller code naming any of them
// compiles. Metadata value types use 0-12; as tensor types the loader reads F32 (6 in the reference's
// convention), FLOAT16 (48), Q4_0, Q4_1 and Q8_0; the other block types are recognised by id and
// rejected when read (-20), as the reference's read_tensor_data does.
enum class GGUFValueType : uint32 {
    UINT8 = 0, INT8 = 1, UINT16 = 2, INT16 = 3, UINT32 = 4, INT32 = 5, FLOAT32 = 6, BOOL = 7,
    STRING = 8, ARRAY = 9, UINT64 = 10, INT64 = 11, FLOAT64 = 12,
    Q4_0 = 13, Q4_1 = 14, Q5_0 = 15, Q5_1 = 16, Q8_0 = 17, Q8_1 = 18,
    Q2_K = 19, Q3_K = 20, Q4_K = 21, Q5_K = 22, Q6_K = 23, Q8_K = 24,
    IQ1_S = 25, IQ1_M = 26, IQ2_XXS = 27, IQ2_XS = 28, IQ3_XXS = 29, IQ4_XS = 30, IQ4_NL = 31,
    IQ5_S = 32, IQ5_M = 33, IQ6_N = 34, IQ6_1 = 35, IQ2_S = 36, IQ3_S = 37, IQ4_1 = 38, IQ3_1 = 39,
    IQ2_1 = 40, IQ1_1 = 41, IQ4_NL_2 = 42, IQ3_L = 43, IQ3_XS = 44, IQ3_M = 45, IQ4_XS_2 = 46,
    BFLOAT16 = 47, FLOAT16 = 48,
    IQ2_M = 49, IQ3_XS_2 = 50, IQ3_L_2 = 51, IQ3_M_2 = 52, IQ4_XS_3 = 53
};

enum class GGUFConvention : int { REFERENCE = 0, GGML = 1 };

struct GGUFHeader {
    uint32 magic = 0;
    uint32 version = 0;
    uint64 tensor_count = 0;
    uint64 metadata_kv_count = 0;
};

struct GGUFTensorInfo {
    std::string name;
    uint32 n_dimensions = 0;
    std::vector<uint64> dimensions;
    GGUFValueType data_type = GGUFValueType::FLOAT32;  // raw id as stored in the file
    uint64 offset = 0;
    uint64 data_offset = 0;  // absolute offset in file
    uint64 data_size = 0;    // bytes of raw data
    bool is_compressed = false;
    uint32 compression_codec = 0;
};

struct GGUFMetadataKV {
    std::string key;
    GGUFValueType value_type = GGUFValueType::UINT8;
    std::vector<uint8_t> raw_value;

    std::string get_string() const;
    uint32_t get_uint32() const;
    int32_t get_int32() const;
    float get_float32() const;
    bool get_bool() const;
    // an array's element bytes (without the u32 element type and u64 count that precede them)
    std::vector<uint8_t> get_array_data() const;
    // an array's element type (UINT8 for a value that is not an array)
    GGUFValueType get_array_element_type() const;
};

// A vocabulary entry of the model file (GGUFLoader.h:110-116): token text and bytes from
// "tokenizer.ggml.tokens", score from "tokenizer.ggml.scores", type from "tokenizer.ggml.token_type".
struct VocabularyEntry {
    std::string token;
    std::vector<uint8_t> bytes;
    float score = 0.0f;
    uint32_t token_type = 0;
    bool is_special = false;
};

// The tokenizer keys of the model file (GGUFLoader.h:119-132), read when the file has a vocabulary.
struct TokenizerConfig {
    std::string model_type = "gpt2";
    bool add_bos_token = false;
    bool add_eos_token = false;
    uint32_t bos_token_id = 0;
    uint32_t eos_token_id = 0;
    uint32_t pad_token_id = 0;
    uint32_t unk_token_id = 0;
    std::string chat_template;
    std::string pre_tokenizer;
    bool add_space_prefix = true;
    bool remove_extra_whitespaces = false;
    std::vector<std::pair<std::string, uint32_t>> added_tokens;
};

// Bounds of the host-side tensor cache behind read_tensor_cached (GGUFLoader.h:135-140).
// enable_compression is accepted and ignored (nothing is compressed here).
struct TensorCacheConfig {
    size_t max_entries = 256;
    size_t max_memory_bytes = 4ULL * 1024 * 1024 * 1024;
    uint64_t ttl_seconds = 300;
    bool enable_compression = true;
};

// Least-recently-used cache of converted tensors (the role of the reference's TensorLRUCache,
// GGUFLoader.h:150-204): bounded by entry count and bytes, entries older than the TTL dropped on
// access.  Thread-safe.
class TensorLRUCache {
   public:
    struct Stats {
        size_t hits = 0;
        size_t misses = 0;
        size_t evictions = 0;
        size_t current_entries = 0;
        size_t current_memory_bytes = 0;
        double hit_rate() const {
            const size_t total = hits + misses;
            return total ? static_cast<double>(hits) / static_cast<double>(total) : 0.0;
        }
    };
    explicit TensorLRUCache(const TensorCacheConfig& config = TensorCacheConfig{});
    bool get(const std::string& name, std::vector<float>& out);
    void put(const std::string& name, const std::vector<float>& data);
    // the reference's signature (the tensor info is not needed to cache the values)
    void put(const std::string& name, const std::vector<float>& data, const GGUFTensorInfo&) { put(name, data); }
    bool contains(const std::string& name) const;
    void clear();
    Stats get_stats() const;
    void touch(const std::string& name);
    size_t remove_expired();
    const TensorCacheConfig& config() const { return config_; }

   private:
    struct Entry {
        std::string name;
        std::vector<float> data;
        std::chrono::steady_clock::time_point stored;
    };
    TensorCacheConfig config_;
    mutable std::mutex mu_;
    std::list<Entry> lru_;  // front = most recently used
    std::unordered_map<std::string, std::list<Entry>::iterator> index_;
    size_t bytes_ = 0;
    Stats stats_;
    bool expired(const Entry& e) const;
    void drop(std::list<Entry>::iterator it, bool eviction);
};

class GGUFLoader {
   public:
    explicit GGUFLoader(const Path& file_path);
    ~GGUFLoader();
    GGUFLoader(const GGUFLoader&) = delete;
    GGUFLoader& operator=(const GGUFLoader&) = delete;

    ExpectedVoid load();
    ExpectedVoid close();

    ModelConfig get_model_config() const;
    std::vector<PackMetadata> generate_packs(const ModelConfig& config);

    uint64 tensor_count() const;
    uint64 metadata_count() const;

    const GGUFTensorInfo* get_tensor(const std::string& name) const;
    Expected<std::vector<float>> read_tensor_data(const GGUFTensorInfo& tensor, bool fp16_to_fp32 = true);
    Expected<std::vector<float>> read_tensor_cached(const std::string& tensor_name, bool fp16_to_fp32 = true);
    std::vector<Expected<std::vector<float>>> read_tensors_parallel(const std::vector<std::string>& tensor_names,
                                                                    bool fp16_to_fp32 = true);

    // Reads every named tensor as read_tensor_data does, spread over num_chunks threads; one result
    // per name in the given order (-30 for a name that is not in the model).  The reference routes this
    // through StreamingTensorReader and drops names it cannot find (GGUFLoader.cpp:1446-1494).
    std::vector<Expected<std::vector<float>>> stream_tensors_parallel(const std::vector<std::string>& tensor_names,
                                                                      uint32_t num_chunks = 4);

    // Vocabulary and tokenizer keys of the file (empty / defaults when it has no "tokenizer.ggml.tokens"
    // array), parsed at load as GGUFLoaderImpl::parse_vocabulary does (GGUFLoader.cpp:982-1075).
    const std::vector<VocabularyEntry>& get_vocabulary() const { return vocabulary_; }
    const TokenizerConfig& get_tokenizer_config() const { return tokenizer_config_; }

    // The cache behind read_tensor_cached (GGUFLoader.cpp:1504-1518).
    void clear_tensor_cache();
    size_t get_tensor_cache_size() const;  // bytes held
    TensorLRUCache::Stats get_cache_stats() const;
    void configure_cache(const TensorCacheConfig& config);  // replaces the cache (entries dropped)

    // Multi-file models: the tensors of another GGUF file join this model's (get_tensor, the tensor
    // names and counts, generate_packs, read_tensor_data, the engine's upload); each file keeps its own
    // tensor-type convention.  Metadata stays this file's.  A name already present is not replaced.
    // Returns the shard's load error, or -60 when this loader is not loaded.  (The reference only logs
    // the path and reports success, GGUFLoader.cpp:1520-1529.)
    ExpectedVoid add_shard(const Path& shard_path);
    bool is_sharded() const { return !shards_.empty(); }

    std::vector<std::string> get_tensor_names() const;
    std::vector<std::string> get_metadata_keys() const;
    const GGUFMetadataKV* get_metadata(const std::string& key) const;

    static uint64 align_offset(uint64 offset, uint64 alignment);
    uint32_t get_version() const { return header_.version; }
    bool is_valid() const { return loaded_; }

    // Additive API used by the HBM pack uploader.
    GGUFConvention convention() const { return convention_; }
    uint64 data_start() const { return data_start_; }
    // VSL_DT_F32 / VSL_DT_F16 for tensors this backend can upload, -1 otherwise
    int storage_dtype(const GGUFTensorInfo& t) const;
    // mapped raw bytes of a tensor (nullptr if out of range)
    const uint8_t* tensor_bytes(const GGUFTensorInfo& t) const;
    // VSL_WF_* storage format of a tensor that vsl_convert_weights can expand (F32, F16, Q4_0, Q4_1,
    // Q8_0), -1 otherwise.  A ggml-id quantized tensor needs ne0 to be a whole number of blocks.
    int weight_format(const GGUFTensorInfo& t) const;
    // VSL_QL_REFERENCE or VSL_QL_GGML: block layout of this file's quantized tensors
    int block_layout() const;
    // the block layout of the file (this one or a shard) holding `t`
    int block_layout(const GGUFTensorInfo& t) const;

   private:
    Path file_path_;
    int fd_ = -1;
    const uint8_t* map_ = nullptr;
    size_t size_ = 0;
    bool loaded_ = false;
    GGUFHeader header_{};
    GGUFConvention convention_ = GGUFConvention::REFERENCE;
    uint64 data_start_ = 0;
    std::unordered_map<std::string, GGUFMetadataKV> metadata_;
    std::vector<std::string> metadata_order_;
    std::unordered_map<std::string, GGUFTensorInfo> tensors_;
    std::vector<std::string> tensor_order_;
    std::unique_ptr<TensorLRUCache> tensor_cache_;
    std::vector<VocabularyEntry> vocabulary_;
    TokenizerConfig tokenizer_config_;
    std::vector<std::unique_ptr<GGUFLoader>> shards_;

    void parse_vocabulary();
    // the shard whose tensor table holds `t` (nullptr: this file's, or unknown)
    const GGUFLoader* shard_of(const GGUFTensorInfo& t) const;
};

// IEEE binary16 <-> binary32 (every case exact / round to nearest even; the reference's
// convert_fp16_to_fp32, GGUFLoader.cpp:1225-1262, gives the same values except for NaN payloads).
float half_to_float(uint16_t h);
uint16_t float_to_half(float f);
// dequantize_tensor (GGUFLoader.cpp:1121-1223) on the host, for read_tensor_data: expands Q4_0 /
// Q4_1 / Q8_0 blocks (fmt = VSL_WF_*) in the given block layout (VSL_QL_*).  Whole blocks are read
// while they fit in src_bytes, the last one possibly partial; returns the number of floats written
// (below n when the data runs out, as the reference's loop guard does).
uint64 dequantize_blocks(const uint8_t* src, uint64 src_bytes, int fmt, int layout, uint64 n, float* out);
// Quantize n floats into ceil(n / 32) blocks of `fmt` (a short last block is zero padded).  Q8_0:
// d = max|x| / 127, q = round(x / d); Q4_0: d = -(the value of largest magnitude) / 8,
// nibble = clamp(floor(x / d + 8.5)); Q4_1: d = (max - min) / 15, m = min,
// nibble = clamp(floor((x - m) / d + 0.5)).  Used for synthetic files and fixtures.
std::vector<uint8_t> quantize_blocks(const float* x, uint64 n, int fmt, int layout);

// Minimal GGUF writer (v3) for synthetic models and fixtures.
class GGUFWriter {
   public:
    explicit GGUFWriter(GGUFConvention conv) : conv_(conv) {}
    void add_u32(const std::string& key, uint32_t v);
    void add_f32(const std::string& key, float v);
    void add_string(const std::string& key, const std::string& v);
    void add_string_array(const std::string& key, const std::vector<std::string>& v);
    void add_bool(const std::string& key, bool v);
    // an array of fixed-size elements: elem_type is the GGUF metadata type id (e.g. 6 FLOAT32, 5 INT32),
    // elems `count` values of `bytes` bytes in total
    void add_array(const std::string& key, uint32_t elem_type, uint64_t count, const void* elems, uint64_t bytes);
    // data: raw bytes in the storage type (is_f16 ? binary16 : binary32); dims ne0-first
    void add_tensor(const std::string& name, const std::vector<uint64_t>& dims, bool is_f16, const void* data,
                    uint64_t bytes);
    // data: raw bytes in storage format fmt (VSL_WF_*: F32, F16, or blocks from quantize_blocks)
    void add_tensor_format(const std::string& name, const std::vector<uint64_t>& dims, int fmt, const void* data,
                           uint64_t bytes);
    ExpectedVoid write(const Path& path) const;

   private:
    struct KV {
        std::string key;
        uint32_t type;
        std::vector<uint8_t> bytes;
    };
    struct T {
        std::string name;
        std::vector<uint64_t> dims;
        int fmt;  // VSL_WF_*
        const void* data;
        uint64_t bytes;
    };
    GGUFConvention conv_;
    std::vector<KV> kvs_;
    std::vector<T> tensors_;
};

}  // namespace vk_symbiote
