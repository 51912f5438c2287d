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

#include <cstdint>
#include <memory>
#include <mutex>
#include <string>
#include <unordered_map>
#include <vector>

#include "Common.h"
#include "NomadPack.h"

namespace vk_symbiote {

enum class GGUFValueType : uint32 {
    UINT8 = 0, INT8 = 1, UINT16 = 2, INT16 = 3, UINT32 = 4, INT32 = 5, FLOAT32 = 6, BOOL = 7,
    STRING = 8, ARRAY = 9, UINT64 = 10, INT64 = 11, FLOAT64 = 12,
    Q4_0 = 13, Q4_1 = 14, Q5_0 = 15, Q5_1 = 16, Q8_0 = 17,
    BFLOAT16 = 47, FLOAT16 = 48
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
    std::vector<uint8_t> get_array_data() const;
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
    std::unordered_map<std::string, std::vector<float>> cache_;
    std::mutex cache_mu_;
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
