// GGUFLoader.cpp -- memory-mapped GGUF reader and a v3 writer.
// Layout and metadata semantics follow the reference's GGUFLoaderImpl
// (vk_symbiote/src/GGUFLoader.cpp:625-663 load, :847-980 metadata / tensor infos / read_value,
// :673-728 get_model_config, :730-751 generate_packs, :1085-1119 sizes, :1225-1262 fp16).
#include "GGUFLoader.h"

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cstdio>
#include <cstring>
#include <fstream>
#include <functional>
#include <future>
#include <thread>

#include "vsl_hip.h"

namespace vk_symbiote {

// ------------------------------------------------------------------------------------------
// metadata accessors (GGUFLoader.cpp:32-66): a value of another type reads as 0 / "" / false
// ------------------------------------------------------------------------------------------
std::string GGUFMetadataKV::get_string() const {
    if (value_type != GGUFValueType::STRING || raw_value.size() < 8) return "";
    uint64_t len;
    std::memcpy(&len, raw_value.data(), 8);
    if (len > raw_value.size() - 8) return "";
    return std::string(reinterpret_cast<const char*>(raw_value.data() + 8), len);
}
uint32_t GGUFMetadataKV::get_uint32() const {
    if (value_type != GGUFValueType::UINT32 || raw_value.size() < 4) return 0;
    uint32_t v;
    std::memcpy(&v, raw_value.data(), 4);
    return v;
}
int32_t GGUFMetadataKV::get_int32() const {
    if (value_type != GGUFValueType::INT32 || raw_value.size() < 4) return 0;
    int32_t v;
    std::memcpy(&v, raw_value.data(), 4);
    return v;
}
float GGUFMetadataKV::get_float32() const {
    if (value_type != GGUFValueType::FLOAT32 || raw_value.size() < 4) return 0.0f;
    float v;
    std::memcpy(&v, raw_value.data(), 4);
    return v;
}
bool GGUFMetadataKV::get_bool() const {
    if (value_type != GGUFValueType::BOOL || raw_value.empty()) return false;
    return raw_value[0] != 0;
}
// arrays are stored as (u32 element type, u64 count, elements); the accessors split that header off
std::vector<uint8_t> GGUFMetadataKV::get_array_data() const {
    if (value_type != GGUFValueType::ARRAY || raw_value.size() < 12) return {};
    return std::vector<uint8_t>(raw_value.begin() + 12, raw_value.end());
}
GGUFValueType GGUFMetadataKV::get_array_element_type() const {
    if (value_type != GGUFValueType::ARRAY || raw_value.size() < 4) return GGUFValueType::UINT8;
    uint32_t t;
    std::memcpy(&t, raw_value.data(), 4);
    return static_cast<GGUFValueType>(t);
}

// ------------------------------------------------------------------------------------------
// parsing
// ------------------------------------------------------------------------------------------
namespace {

struct Cursor {
    const uint8_t* p;
    const uint8_t* end;
    bool take(void* dst, size_t n) {
        if (static_cast<size_t>(end - p) < n) return false;
        if (dst) std::memcpy(dst, p, n);
        p += n;
        return true;
    }
};

// read_value (GGUFLoader.cpp:913-980): raw_value holds scalars as bytes, strings as
// (u64 len, bytes), arrays as (u32 elem type, u64 count, elements...)
bool read_value(Cursor& c, uint32_t type, std::vector<uint8_t>& out, int depth) {
    if (depth > 4) return false;
    auto take_n = [&](size_t n) {
        size_t o = out.size();
        out.resize(o + n);
        return c.take(out.data() + o, n);
    };
    switch (type) {
        case 0: case 1: case 7: return take_n(1);
        case 2: case 3: return take_n(2);
        case 4: case 5: case 6: return take_n(4);
        case 10: case 11: case 12: return take_n(8);
        case 8: {
            uint64_t len;
            if (!c.take(&len, 8) || len > static_cast<uint64_t>(c.end - c.p)) return false;
            size_t o = out.size();
            out.resize(o + 8);
            std::memcpy(out.data() + o, &len, 8);
            return take_n(len);
        }
        case 9: {
            uint32_t et;
            uint64_t cnt;
            if (!c.take(&et, 4) || !c.take(&cnt, 8)) return false;
            size_t o = out.size();
            out.resize(o + 12);
            std::memcpy(out.data() + o, &et, 4);
            std::memcpy(out.data() + o + 4, &cnt, 8);
            for (uint64_t i = 0; i < cnt; ++i)
                if (!read_value(c, et, out, depth + 1)) return false;
            return true;
        }
        default: return false;
    }
}

uint64_t reference_type_size(uint32_t t, uint64_t n) {  // calculate_tensor_data_size :1085-1119
    switch (t) {
        case 0: case 1: return n;
        case 2: case 3: case 47: case 48: return n * 2;
        case 4: case 5: case 6: return n * 4;
        case 10: case 11: case 12: return n * 8;
        case 13: return (n / 32) * 18 + ((n % 32) ? 18 : 0);
        case 14: return (n / 32) * 20 + ((n % 32) ? 20 : 0);
        case 15: return (n / 32) * 22 + ((n % 32) ? 22 : 0);
        case 16: return (n / 32) * 24 + ((n % 32) ? 24 : 0);
        case 17: return (n / 32) * 34 + ((n % 32) ? 34 : 0);
        default: return n * 4;
    }
}

uint64_t ggml_type_size(uint32_t t, uint64_t n) {
    switch (t) {
        case 0: return n * 4;
        case 1: return n * 2;
        case 2: return (n / 32) * 18;
        case 3: return (n / 32) * 20;
        case 8: return (n / 32) * 34;
        case 30: return n * 2;
        default: return 0;
    }
}

// The scale helper local to dequantize_tensor (GGUFLoader.cpp:1132-1149).  Where the exponent
// field is 0 it returns ldexp(mantissa, -24) with no sign (so -0 reads as +0 and a negative
// subnormal as positive); every other pattern converts exactly.
float reference_block_scale(uint16_t h) {
    if (((h >> 10) & 0x1F) == 0) return static_cast<float>(h & 0x3FF) * 5.9604644775390625e-08f;
    return half_to_float(h);
}

constexpr uint64_t kBlock = 32;

uint64_t block_bytes(int fmt) {
    return fmt == VSL_WF_Q4_0 ? 18 : fmt == VSL_WF_Q4_1 ? 20 : fmt == VSL_WF_Q8_0 ? 34 : 0;
}

// element index held by nibble `hi` (0 low, 1 high) of byte i in a 4-bit block
inline uint32_t nibble_element(uint32_t i, uint32_t hi, bool ref_layout) {
    return ref_layout ? 2 * i + hi : i + 16 * hi;
}

}  // namespace

float half_to_float(uint16_t h) {
    uint32_t sign = static_cast<uint32_t>(h >> 15) << 31, e = (h >> 10) & 0x1F, m = h & 0x3FF, bits;
    if (e == 0) {
        if (m == 0) {
            bits = sign;
        } else {
            float v = static_cast<float>(m) * 5.9604644775390625e-08f;
            std::memcpy(&bits, &v, 4);
            bits |= sign;
        }
    } else if (e == 31) {
        bits = sign | 0x7F800000u | (m << 13);
    } else {
        bits = sign | ((e + 112u) << 23) | (m << 13);
    }
    float f;
    std::memcpy(&f, &bits, 4);
    return f;
}

uint16_t float_to_half(float f) {  // round to nearest even
    uint32_t x;
    std::memcpy(&x, &f, 4);
    uint32_t sign = (x >> 16) & 0x8000u, a = x & 0x7FFFFFFFu;
    if (a >= 0x7F800000u) return (uint16_t)(sign | 0x7C00u | ((a & 0x7FFFFFu) ? (0x200u | ((a & 0x7FFFFFu) >> 13)) : 0));
    if (a >= 0x477FF000u) return (uint16_t)(sign | 0x7C00u);
    if (a < 0x38800000u) {
        if (a < 0x33000000u) return (uint16_t)sign;
        uint32_t e = a >> 23, m = (a & 0x7FFFFFu) | 0x800000u, sh = 126 - e;
        uint32_t q = m >> sh, rem = m & ((1u << sh) - 1), half = 1u << (sh - 1);
        if (rem > half || (rem == half && (q & 1))) q++;
        return (uint16_t)(sign | q);
    }
    uint32_t q = (((a >> 23) - 112) << 10) | ((a & 0x7FFFFFu) >> 13), rem = a & 0x1FFFu;
    if (rem > 0x1000u || (rem == 0x1000u && (q & 1))) q++;
    return (uint16_t)(sign | q);
}

uint64 dequantize_blocks(const uint8_t* src, uint64 src_bytes, int fmt, int layout, uint64 n, float* out) {
    const uint64_t bb = block_bytes(fmt);
    if (!bb) return 0;
    const bool ref = layout == VSL_QL_REFERENCE;
    auto scale = [&](const uint8_t* p) {
        uint16_t h;
        std::memcpy(&h, p, 2);
        return ref ? reference_block_scale(h) : half_to_float(h);
    };
    uint64_t done = 0;
    for (uint64_t b = 0; done < n && (b + 1) * bb <= src_bytes; ++b) {
        const uint8_t* blk = src + b * bb;
        const uint64_t cnt = std::min<uint64_t>(kBlock, n - done);
        float v[kBlock];
        const float d = scale(blk);
        if (fmt == VSL_WF_Q8_0) {
            for (uint32_t j = 0; j < kBlock; ++j) v[j] = static_cast<float>(static_cast<int8_t>(blk[2 + j])) * d;
        } else {
            // Q4_0 is (nibble - 8) * d with no addend: adding +0 would turn a -0 product into +0
            const bool with_min = fmt == VSL_WF_Q4_1;
            const float m = with_min ? scale(blk + 2) : 0.0f;
            const uint8_t* qs = blk + (with_min ? 4 : 2);
            for (uint32_t i = 0; i < 16; ++i)
                for (uint32_t hi = 0; hi < 2; ++hi) {
                    const int nib = (qs[i] >> (4 * hi)) & 15;
                    v[nibble_element(i, hi, ref)] =
                        with_min ? static_cast<float>(nib) * d + m : static_cast<float>(nib - 8) * d;
                }
        }
        std::memcpy(out + done, v, cnt * sizeof(float));
        done += cnt;
    }
    return done;
}

std::vector<uint8_t> quantize_blocks(const float* x, uint64 n, int fmt, int layout) {
    const uint64_t bb = block_bytes(fmt), nb = (n + kBlock - 1) / kBlock;
    std::vector<uint8_t> out(nb * bb, 0);
    if (!bb) return {};
    const bool ref = layout == VSL_QL_REFERENCE;
    // blocks are independent: contiguous ranges of them on up to 32 threads
    auto quantize_range = [&](uint64_t b0, uint64_t b1) {
        for (uint64_t b = b0; b < b1; ++b) {
            float v[kBlock] = {0};
            const uint64_t cnt = std::min<uint64_t>(kBlock, n - b * kBlock);
            std::memcpy(v, x + b * kBlock, cnt * sizeof(float));
            uint8_t* blk = out.data() + b * bb;
            auto put_half = [](uint8_t* p, float f) {
                const uint16_t h = float_to_half(f);
                std::memcpy(p, &h, 2);
                return half_to_float(h);  // the scale the reader will see
            };
            if (fmt == VSL_WF_Q8_0) {
                float amax = 0.0f;
                for (float f : v) amax = std::max(amax, std::fabs(f));
                const float d = put_half(blk, amax / 127.0f);
                const float inv = d != 0.0f ? 1.0f / d : 0.0f;
                for (uint32_t j = 0; j < kBlock; ++j) {
                    const float q = std::nearbyint(v[j] * inv);
                    blk[2 + j] = static_cast<uint8_t>(static_cast<int8_t>(std::min(127.0f, std::max(-128.0f, q))));
                }
                continue;
            }
            uint8_t nib[kBlock];
            if (fmt == VSL_WF_Q4_0) {
                float ext = 0.0f;
                for (float f : v)
                    if (std::fabs(f) > std::fabs(ext)) ext = f;
                const float d = put_half(blk, ext / -8.0f);
                const float inv = d != 0.0f ? 1.0f / d : 0.0f;
                for (uint32_t j = 0; j < kBlock; ++j)
                    nib[j] = static_cast<uint8_t>(std::min(15.0f, std::max(0.0f, std::floor(v[j] * inv + 8.5f))));
            } else {
                float lo = v[0], hi = v[0];
                for (float f : v) { lo = std::min(lo, f); hi = std::max(hi, f); }
                const float d = put_half(blk, (hi - lo) / 15.0f);
                const float m = put_half(blk + 2, lo);
                const float inv = d != 0.0f ? 1.0f / d : 0.0f;
                for (uint32_t j = 0; j < kBlock; ++j)
                    nib[j] = static_cast<uint8_t>(std::min(15.0f, std::max(0.0f, std::floor((v[j] - m) * inv + 0.5f))));
            }
            uint8_t* qs = blk + (fmt == VSL_WF_Q4_1 ? 4 : 2);
            for (uint32_t i = 0; i < 16; ++i)
                qs[i] = static_cast<uint8_t>(nib[nibble_element(i, 0, ref)] | (nib[nibble_element(i, 1, ref)] << 4));
        }
    };
    unsigned nt = std::max(1u, std::min(32u, std::thread::hardware_concurrency()));
    if (nb < 16384) nt = 1;
    std::vector<std::thread> th;
    for (unsigned t = 1; t < nt; ++t) th.emplace_back(quantize_range, nb * t / nt, nb * (t + 1) / nt);
    quantize_range(0, nb / nt);
    for (auto& t : th) t.join();
    return out;
}

GGUFLoader::GGUFLoader(const Path& file_path)
    : file_path_(file_path), tensor_cache_(std::make_unique<TensorLRUCache>()) {}
GGUFLoader::~GGUFLoader() { close(); }

uint64 GGUFLoader::align_offset(uint64 offset, uint64 alignment) {
    if (alignment == 0) return offset;
    return (offset + alignment - 1) / alignment * alignment;
}

ExpectedVoid GGUFLoader::close() {
    if (map_) munmap(const_cast<uint8_t*>(map_), size_);
    if (fd_ >= 0) ::close(fd_);
    map_ = nullptr;
    fd_ = -1;
    size_ = 0;
    loaded_ = false;
    metadata_.clear();
    metadata_order_.clear();
    tensors_.clear();
    tensor_order_.clear();
    if (tensor_cache_) tensor_cache_->clear();
    vocabulary_.clear();
    tokenizer_config_ = TokenizerConfig{};
    shards_.clear();
    return ExpectedVoid();
}

ExpectedVoid GGUFLoader::load() {
    close();
    fd_ = ::open(file_path_.c_str(), O_RDONLY);
    if (fd_ < 0) return kErrOpen;
    struct stat st;
    if (fstat(fd_, &st) != 0) { close(); return kErrOpen; }
    size_ = static_cast<size_t>(st.st_size);
    if (size_ < sizeof(GGUFHeader)) { close(); return kErrMagic; }
    void* m = mmap(nullptr, size_, PROT_READ, MAP_PRIVATE, fd_, 0);
    if (m == MAP_FAILED) { close(); return kErrOpen; }
    map_ = static_cast<const uint8_t*>(m);
    Cursor c{map_, map_ + size_};
    c.take(&header_.magic, 4);
    if (header_.magic != 0x46554747u) { close(); return kErrMagic; }
    c.take(&header_.version, 4);
    c.take(&header_.tensor_count, 8);
    c.take(&header_.metadata_kv_count, 8);
    if (header_.metadata_kv_count > size_ / 12 || header_.tensor_count > size_ / 24) { close(); return kErrMetadata; }
    for (uint64_t i = 0; i < header_.metadata_kv_count; ++i) {  // parse_metadata :847-874
        uint64_t klen;
        if (!c.take(&klen, 8) || klen > static_cast<uint64_t>(c.end - c.p)) { close(); return kErrMetadata; }
        GGUFMetadataKV kv;
        kv.key.assign(reinterpret_cast<const char*>(c.p), klen);
        c.p += klen;
        uint32_t vt;
        if (!c.take(&vt, 4)) { close(); return kErrMetadata; }
        kv.value_type = static_cast<GGUFValueType>(vt);
        if (!read_value(c, vt, kv.raw_value, 0)) { close(); return kErrMetadata; }
        if (!metadata_.count(kv.key)) metadata_order_.push_back(kv.key);
        metadata_[kv.key] = std::move(kv);
    }
    for (uint64_t i = 0; i < header_.tensor_count; ++i) {  // parse_tensor_info :876-911
        GGUFTensorInfo info;
        uint64_t nlen;
        if (!c.take(&nlen, 8) || nlen > static_cast<uint64_t>(c.end - c.p)) { close(); return kErrTensorInfo; }
        info.name.assign(reinterpret_cast<const char*>(c.p), nlen);
        c.p += nlen;
        if (!c.take(&info.n_dimensions, 4) || info.n_dimensions > 8) { close(); return kErrTensorInfo; }
        info.dimensions.resize(info.n_dimensions);
        for (uint32_t d = 0; d < info.n_dimensions; ++d)
            if (!c.take(&info.dimensions[d], 8)) { close(); return kErrTensorInfo; }
        uint32_t dt;
        if (!c.take(&dt, 4) || !c.take(&info.offset, 8)) { close(); return kErrTensorInfo; }
        info.data_type = static_cast<GGUFValueType>(dt);
        if (!tensors_.count(info.name)) tensor_order_.push_back(info.name);
        tensors_[info.name] = std::move(info);
    }
    const uint64_t after_infos = static_cast<uint64_t>(c.p - map_);

    convention_ = GGUFConvention::REFERENCE;
    if (auto* kv = get_metadata("vsl.tensor_type_convention")) {
        convention_ = kv->get_string() == "ggml" ? GGUFConvention::GGML : GGUFConvention::REFERENCE;
    } else if (get_metadata("general.alignment")) {
        convention_ = GGUFConvention::GGML;
    } else {
        bool has_ggml = false, has_ref = false;
        for (auto& kv : tensors_) {
            uint32_t t = static_cast<uint32_t>(kv.second.data_type);
            if (t == 0 || t == 1 || t == 2 || t == 3 || t == 8) has_ggml = true;
            if (t == 48) has_ref = true;
        }
        convention_ = (has_ggml && !has_ref) ? GGUFConvention::GGML : GGUFConvention::REFERENCE;
    }
    if (convention_ == GGUFConvention::REFERENCE) {
        data_start_ = after_infos;  // GGUFLoader.cpp:653
    } else {
        uint64_t align = 32;
        if (auto* kv = get_metadata("general.alignment"))
            if (kv->get_uint32()) align = kv->get_uint32();
        data_start_ = align_offset(after_infos, align);
    }
    for (auto& kv : tensors_) {
        GGUFTensorInfo& t = kv.second;
        // The file is untrusted: an element count whose byte size cannot be represented is a malformed
        // tensor info (the largest element is 8 bytes, so counts stay below 2^60).
        uint64_t n = 1;
        for (auto d : t.dimensions)
            if (__builtin_mul_overflow(n, d, &n) || n >= (1ull << 60)) { close(); return kErrTensorInfo; }
        // an offset that wraps past 2^64 saturates; tensor_bytes() then rejects it like any other
        // range outside the mapping
        if (__builtin_add_overflow(data_start_, t.offset, &t.data_offset)) t.data_offset = UINT64_MAX;
        t.data_size = convention_ == GGUFConvention::REFERENCE ? reference_type_size(static_cast<uint32_t>(t.data_type), n)
                                                               : ggml_type_size(static_cast<uint32_t>(t.data_type), n);
    }
    parse_vocabulary();
    loaded_ = true;
    return ExpectedVoid();
}

ModelConfig GGUFLoader::get_model_config() const {  // GGUFLoader.cpp:673-728
    ModelConfig c;
    if (auto* kv = get_metadata("llama.embedding_length")) c.hidden_size = kv->get_uint32();
    else if (auto* kv2 = get_metadata("general.embedding_length")) c.hidden_size = kv2->get_uint32();
    if (auto* kv = get_metadata("llama.block_count")) c.num_layers = kv->get_uint32();
    else if (auto* kv2 = get_metadata("general.block_count")) c.num_layers = kv2->get_uint32();
    if (auto* kv = get_metadata("llama.attention.head_count")) c.num_attention_heads = kv->get_uint32();
    if (auto* kv = get_metadata("llama.attention.head_count_kv")) c.num_key_value_heads = kv->get_uint32();
    else c.num_key_value_heads = c.num_attention_heads;
    if (auto* kv = get_metadata("llama.feed_forward_length")) c.intermediate_size = kv->get_uint32();
    if (auto* kv = get_metadata("llama.vocab_size")) {
        c.vocab_size = kv->get_uint32();
    } else if (auto* kv2 = get_metadata("tokenizer.ggml.tokens")) {
        // the array's element count (the u64 after its element type)
        if (kv2->value_type == GGUFValueType::ARRAY && kv2->raw_value.size() >= 12) {
            uint64_t cnt;
            std::memcpy(&cnt, kv2->raw_value.data() + 4, 8);
            c.vocab_size = static_cast<uint32_t>(cnt);
        }
    }
    if (auto* kv = get_metadata("llama.rope.freq_base")) c.rope_theta = kv->get_float32();
    if (auto* kv = get_metadata("llama.context_length")) c.max_position_embeddings = kv->get_uint32();
    if (auto* kv = get_metadata("general.architecture")) c.model_type = kv->get_string();
    if (auto* kv = get_metadata("llama.attention.layer_norm_rms_epsilon"))
        if (kv->value_type == GGUFValueType::FLOAT32) c.rms_epsilon = kv->get_float32();
    c.head_dim = c.num_attention_heads ? c.hidden_size / c.num_attention_heads : 0;
    if (const GGUFTensorInfo* q = get_tensor("blk.0.attn_q.weight")) c.use_fp16 = storage_dtype(*q) == VSL_DT_F16;
    return c;
}

std::vector<PackMetadata> GGUFLoader::generate_packs(const ModelConfig&) {  // GGUFLoader.cpp:730-751
    std::vector<PackMetadata> packs;
    const std::vector<std::string> names = get_tensor_names();
    packs.reserve(names.size());
    for (const auto& name : names) {
        const GGUFTensorInfo& info = *get_tensor(name);
        PackMetadata p;
        p.pack_id = std::hash<std::string>{}(name);
        p.tensor_name = name;
        p.layer_idx = extract_layer_index(name);
        p.head_idx = 0;
        p.compressed_size = info.data_size;
        p.decompressed_size = info.data_size;
        p.file_offset = info.data_offset;
        p.base_priority = calculate_pack_priority(name);
        p.type = classify_tensor_type(name);
        p.alignment = 256;
        p.n_dimensions = info.n_dimensions;
        p.dimensions = info.dimensions;
        packs.push_back(std::move(p));
    }
    return packs;
}

uint64 GGUFLoader::tensor_count() const {
    uint64 n = header_.tensor_count;
    for (const auto& sh : shards_) n += sh->tensor_count();
    return n;
}
uint64 GGUFLoader::metadata_count() const { return header_.metadata_kv_count; }

const GGUFTensorInfo* GGUFLoader::get_tensor(const std::string& name) const {
    auto it = tensors_.find(name);
    if (it != tensors_.end()) return &it->second;
    for (const auto& sh : shards_)
        if (const GGUFTensorInfo* t = sh->get_tensor(name)) return t;
    return nullptr;
}

const GGUFLoader* GGUFLoader::shard_of(const GGUFTensorInfo& t) const {
    auto it = tensors_.find(t.name);
    if (it != tensors_.end() && &it->second == &t) return nullptr;
    for (const auto& sh : shards_) {
        auto jt = sh->tensors_.find(t.name);
        if (jt != sh->tensors_.end() && &jt->second == &t) return sh.get();
    }
    return nullptr;
}

int GGUFLoader::storage_dtype(const GGUFTensorInfo& t) const {
    if (const GGUFLoader* sh = shard_of(t)) return sh->storage_dtype(t);
    const uint32_t id = static_cast<uint32_t>(t.data_type);
    if (convention_ == GGUFConvention::REFERENCE) {
        if (id == 6) return VSL_DT_F32;
        if (id == 48) return VSL_DT_F16;
        return -1;
    }
    if (id == 0) return VSL_DT_F32;
    if (id == 1) return VSL_DT_F16;
    return -1;
}

int GGUFLoader::weight_format(const GGUFTensorInfo& t) const {
    if (const GGUFLoader* sh = shard_of(t)) return sh->weight_format(t);
    const uint32_t id = static_cast<uint32_t>(t.data_type);
    if (convention_ == GGUFConvention::REFERENCE) {
        switch (id) {
            case 6: return VSL_WF_F32;
            case 48: return VSL_WF_F16;
            case 13: return VSL_WF_Q4_0;
            case 14: return VSL_WF_Q4_1;
            case 17: return VSL_WF_Q8_0;
            default: return -1;
        }
    }
    switch (id) {
        case 0: return VSL_WF_F32;
        case 1: return VSL_WF_F16;
        case 2: case 3: case 8:
            // ggml never splits a block across rows
            if (t.dimensions.empty() || t.dimensions[0] % kBlock) return -1;
            return id == 2 ? VSL_WF_Q4_0 : (id == 3 ? VSL_WF_Q4_1 : VSL_WF_Q8_0);
        default: return -1;
    }
}

int GGUFLoader::block_layout() const {
    return convention_ == GGUFConvention::GGML ? VSL_QL_GGML : VSL_QL_REFERENCE;
}

int GGUFLoader::block_layout(const GGUFTensorInfo& t) const {
    const GGUFLoader* sh = shard_of(t);
    return sh ? sh->block_layout() : block_layout();
}

const uint8_t* GGUFLoader::tensor_bytes(const GGUFTensorInfo& t) const {
    if (const GGUFLoader* sh = shard_of(t)) return sh->tensor_bytes(t);
    // written so that no sum can wrap: [data_offset, data_offset + data_size) inside the data section
    if (!map_ || t.data_offset < data_start_ || t.data_offset > size_ || t.data_size > size_ - t.data_offset)
        return nullptr;
    return map_ + t.data_offset;
}

Expected<std::vector<float>> GGUFLoader::read_tensor_data(const GGUFTensorInfo& t, bool fp16_to_fp32) {
    if (!loaded_) return -10;
    if (const GGUFLoader* sh = shard_of(t)) return const_cast<GGUFLoader*>(sh)->read_tensor_data(t, fp16_to_fp32);
    const uint8_t* p = tensor_bytes(t);
    if (!p) return kErrRead;
    const int dt = storage_dtype(t);
    if (dt == VSL_DT_F32) {
        std::vector<float> r(t.data_size / 4);
        std::memcpy(r.data(), p, r.size() * 4);
        return r;
    }
    if (dt == VSL_DT_F16 && fp16_to_fp32) {
        std::vector<float> r(t.data_size / 2);
        for (size_t i = 0; i < r.size(); ++i) {
            uint16_t h;
            std::memcpy(&h, p + 2 * i, 2);
            r[i] = half_to_float(h);
        }
        return r;
    }
    const int wf = weight_format(t);
    if (wf >= VSL_WF_Q4_0) {  // read_tensor_data -> dequantize_tensor (:775-777)
        uint64_t n = 1;
        for (auto x : t.dimensions) n *= x;
        std::vector<float> r(n);
        r.resize(dequantize_blocks(p, t.data_size, wf, block_layout(), n, r.data()));
        return r;
    }
    const uint32_t id = static_cast<uint32_t>(t.data_type);
    if (convention_ == GGUFConvention::REFERENCE ? (id >= 13 && id <= 53) : (id >= 2 && id != 30))
        return kErrUnsupportedQuant;
    return kErrUnsupportedType;
}

Expected<std::vector<float>> GGUFLoader::read_tensor_cached(const std::string& name, bool fp16_to_fp32) {
    std::vector<float> hit;
    if (tensor_cache_->get(name, hit)) return hit;
    const GGUFTensorInfo* t = get_tensor(name);
    if (!t) return kErrNotFound;
    auto r = read_tensor_data(*t, fp16_to_fp32);
    if (r.has_value()) tensor_cache_->put(name, r.value());
    return r;
}

std::vector<Expected<std::vector<float>>> GGUFLoader::stream_tensors_parallel(const std::vector<std::string>& names,
                                                                              uint32_t num_chunks) {
    std::vector<Expected<std::vector<float>>> out(names.size(), Expected<std::vector<float>>(kErrNotFound));
    const size_t nt = std::max<size_t>(1, std::min<size_t>(num_chunks ? num_chunks : 1, names.size()));
    std::vector<std::thread> th;
    th.reserve(nt);
    for (size_t w = 0; w < nt; ++w)
        th.emplace_back([&, w]() {
            // chunk w: a contiguous range of the names; every slot is written by exactly one thread
            for (size_t i = names.size() * w / nt; i < names.size() * (w + 1) / nt; ++i)
                if (const GGUFTensorInfo* t = get_tensor(names[i])) out[i] = read_tensor_data(*t, true);
        });
    for (auto& t : th) t.join();
    return out;
}

void GGUFLoader::clear_tensor_cache() { tensor_cache_->clear(); }
size_t GGUFLoader::get_tensor_cache_size() const { return tensor_cache_->get_stats().current_memory_bytes; }
TensorLRUCache::Stats GGUFLoader::get_cache_stats() const { return tensor_cache_->get_stats(); }
void GGUFLoader::configure_cache(const TensorCacheConfig& config) { tensor_cache_ = std::make_unique<TensorLRUCache>(config); }

ExpectedVoid GGUFLoader::add_shard(const Path& shard_path) {
    if (!loaded_) return kErrInvalid;
    auto sh = std::make_unique<GGUFLoader>(shard_path);
    ExpectedVoid r = sh->load();
    if (!r.has_value()) return r;
    shards_.push_back(std::move(sh));
    return ExpectedVoid();
}

// GGUFLoaderImpl::parse_vocabulary (GGUFLoader.cpp:982-1075): the tokenizer keys, then the token
// strings of the "tokenizer.ggml.tokens" array with their scores and types where present.
void GGUFLoader::parse_vocabulary() {
    vocabulary_.clear();
    tokenizer_config_ = TokenizerConfig{};
    const GGUFMetadataKV* tokens = get_metadata("tokenizer.ggml.tokens");
    if (!tokens) return;
    if (auto* kv = get_metadata("tokenizer.ggml.model")) tokenizer_config_.model_type = kv->get_string();
    if (auto* kv = get_metadata("tokenizer.ggml.bos_token_id")) tokenizer_config_.bos_token_id = kv->get_uint32();
    if (auto* kv = get_metadata("tokenizer.ggml.eos_token_id")) tokenizer_config_.eos_token_id = kv->get_uint32();
    if (auto* kv = get_metadata("tokenizer.ggml.padding_token_id")) tokenizer_config_.pad_token_id = kv->get_uint32();
    if (auto* kv = get_metadata("tokenizer.ggml.unknown_token_id")) tokenizer_config_.unk_token_id = kv->get_uint32();
    if (auto* kv = get_metadata("tokenizer.ggml.add_bos_token")) tokenizer_config_.add_bos_token = kv->get_bool();
    if (auto* kv = get_metadata("tokenizer.ggml.add_eos_token")) tokenizer_config_.add_eos_token = kv->get_bool();
    if (auto* kv = get_metadata("tokenizer.chat_template")) tokenizer_config_.chat_template = kv->get_string();
    // array payload: element type (u32), count (u64), then the elements
    auto array_view = [](const GGUFMetadataKV* kv, uint32_t want_type, uint64_t& count) -> const std::vector<uint8_t>* {
        if (!kv || kv->value_type != GGUFValueType::ARRAY || kv->raw_value.size() < 12) return nullptr;
        uint32_t et;
        std::memcpy(&et, kv->raw_value.data(), 4);
        std::memcpy(&count, kv->raw_value.data() + 4, 8);
        return et == want_type ? &kv->raw_value : nullptr;
    };
    uint64_t n = 0;
    const std::vector<uint8_t>* a = array_view(tokens, 8, n);
    if (!a) return;
    size_t off = 12;
    for (uint64_t i = 0; i < n; ++i) {
        uint64_t len;
        if (a->size() - off < 8) break;
        std::memcpy(&len, a->data() + off, 8);
        off += 8;
        if (len > a->size() - off) break;
        VocabularyEntry e;
        e.bytes.assign(a->data() + off, a->data() + off + len);
        e.token.assign(reinterpret_cast<const char*>(a->data() + off), len);
        vocabulary_.push_back(std::move(e));
        off += len;
    }
    uint64_t ns = 0;
    if (const std::vector<uint8_t>* sc = array_view(get_metadata("tokenizer.ggml.scores"), 6, ns))
        for (uint64_t i = 0; i < ns && i < vocabulary_.size() && 12 + 4 * (i + 1) <= sc->size(); ++i)
            std::memcpy(&vocabulary_[i].score, sc->data() + 12 + 4 * i, 4);
    uint64_t ny = 0;
    const GGUFMetadataKV* ty = get_metadata("tokenizer.ggml.token_type");
    const std::vector<uint8_t>* tv = array_view(ty, 5, ny);  // INT32 in llama.cpp files
    if (!tv) tv = array_view(ty, 4, ny);                     // UINT32
    if (tv)
        for (uint64_t i = 0; i < ny && i < vocabulary_.size() && 12 + 4 * (i + 1) <= tv->size(); ++i)
            std::memcpy(&vocabulary_[i].token_type, tv->data() + 12 + 4 * i, 4);
}

// ------------------------------------------------------------------------------------------
// TensorLRUCache
// ------------------------------------------------------------------------------------------
TensorLRUCache::TensorLRUCache(const TensorCacheConfig& config) : config_(config) {}

bool TensorLRUCache::expired(const Entry& e) const {
    return config_.ttl_seconds && std::chrono::steady_clock::now() - e.stored > std::chrono::seconds(config_.ttl_seconds);
}

void TensorLRUCache::drop(std::list<Entry>::iterator it, bool eviction) {
    bytes_ -= it->data.size() * sizeof(float);
    index_.erase(it->name);
    lru_.erase(it);
    if (eviction) ++stats_.evictions;
}

bool TensorLRUCache::get(const std::string& name, std::vector<float>& out) {
    std::lock_guard<std::mutex> lk(mu_);
    auto it = index_.find(name);
    if (it == index_.end() || expired(*it->second)) {
        if (it != index_.end()) drop(it->second, true);
        ++stats_.misses;
        return false;
    }
    lru_.splice(lru_.begin(), lru_, it->second);
    out = it->second->data;
    ++stats_.hits;
    return true;
}

void TensorLRUCache::put(const std::string& name, const std::vector<float>& data) {
    const size_t cost = data.size() * sizeof(float);
    std::lock_guard<std::mutex> lk(mu_);
    auto it = index_.find(name);
    if (it != index_.end()) drop(it->second, false);
    if (cost > config_.max_memory_bytes || config_.max_entries == 0) return;  // never fits
    while (!lru_.empty() && (lru_.size() + 1 > config_.max_entries || bytes_ + cost > config_.max_memory_bytes))
        drop(std::prev(lru_.end()), true);
    lru_.push_front(Entry{name, data, std::chrono::steady_clock::now()});
    index_[name] = lru_.begin();
    bytes_ += cost;
}

bool TensorLRUCache::contains(const std::string& name) const {
    std::lock_guard<std::mutex> lk(mu_);
    auto it = index_.find(name);
    return it != index_.end() && !expired(*it->second);
}

void TensorLRUCache::clear() {
    std::lock_guard<std::mutex> lk(mu_);
    lru_.clear();
    index_.clear();
    bytes_ = 0;
}

TensorLRUCache::Stats TensorLRUCache::get_stats() const {
    std::lock_guard<std::mutex> lk(mu_);
    Stats s = stats_;
    s.current_entries = lru_.size();
    s.current_memory_bytes = bytes_;
    return s;
}

void TensorLRUCache::touch(const std::string& name) {
    std::lock_guard<std::mutex> lk(mu_);
    auto it = index_.find(name);
    if (it == index_.end()) return;
    it->second->stored = std::chrono::steady_clock::now();
    lru_.splice(lru_.begin(), lru_, it->second);
}

size_t TensorLRUCache::remove_expired() {
    std::lock_guard<std::mutex> lk(mu_);
    size_t n = 0;
    for (auto it = lru_.begin(); it != lru_.end();) {
        auto nx = std::next(it);
        if (expired(*it)) {
            drop(it, true);
            ++n;
        }
        it = nx;
    }
    return n;
}

std::vector<Expected<std::vector<float>>> GGUFLoader::read_tensors_parallel(const std::vector<std::string>& names,
                                                                            bool fp16_to_fp32) {
    std::vector<std::future<Expected<std::vector<float>>>> fs;
    fs.reserve(names.size());
    for (const auto& n : names)
        fs.push_back(std::async(std::launch::async, [this, n, fp16_to_fp32]() -> Expected<std::vector<float>> {
            const GGUFTensorInfo* t = get_tensor(n);
            if (!t) return kErrNotFound;
            return read_tensor_data(*t, fp16_to_fp32);
        }));
    std::vector<Expected<std::vector<float>>> out;
    out.reserve(names.size());
    for (auto& f : fs) out.push_back(f.get());
    return out;
}

std::vector<std::string> GGUFLoader::get_tensor_names() const {
    std::vector<std::string> names = tensor_order_;
    for (const auto& sh : shards_)
        for (const auto& n : sh->get_tensor_names())
            if (get_tensor(n) == sh->get_tensor(n)) names.push_back(n);  // not shadowed by an earlier file
    return names;
}
std::vector<std::string> GGUFLoader::get_metadata_keys() const { return metadata_order_; }
const GGUFMetadataKV* GGUFLoader::get_metadata(const std::string& key) const {
    auto it = metadata_.find(key);
    return it == metadata_.end() ? nullptr : &it->second;
}

// ------------------------------------------------------------------------------------------
// writer
// ------------------------------------------------------------------------------------------
void GGUFWriter::add_u32(const std::string& key, uint32_t v) {
    KV kv{key, 4, std::vector<uint8_t>(4)};
    std::memcpy(kv.bytes.data(), &v, 4);
    kvs_.push_back(std::move(kv));
}
void GGUFWriter::add_f32(const std::string& key, float v) {
    KV kv{key, 6, std::vector<uint8_t>(4)};
    std::memcpy(kv.bytes.data(), &v, 4);
    kvs_.push_back(std::move(kv));
}
void GGUFWriter::add_string(const std::string& key, const std::string& v) {
    KV kv{key, 8, std::vector<uint8_t>(8 + v.size())};
    uint64_t l = v.size();
    std::memcpy(kv.bytes.data(), &l, 8);
    std::memcpy(kv.bytes.data() + 8, v.data(), v.size());
    kvs_.push_back(std::move(kv));
}
void GGUFWriter::add_bool(const std::string& key, bool v) { kvs_.push_back(KV{key, 7, {static_cast<uint8_t>(v ? 1 : 0)}}); }
void GGUFWriter::add_array(const std::string& key, uint32_t elem_type, uint64_t count, const void* elems,
                           uint64_t bytes) {
    KV kv{key, 9, std::vector<uint8_t>(12 + bytes)};
    std::memcpy(kv.bytes.data(), &elem_type, 4);
    std::memcpy(kv.bytes.data() + 4, &count, 8);
    if (bytes) std::memcpy(kv.bytes.data() + 12, elems, bytes);
    kvs_.push_back(std::move(kv));
}
void GGUFWriter::add_string_array(const std::string& key, const std::vector<std::string>& v) {
    KV kv{key, 9, std::vector<uint8_t>(12)};
    const uint32_t et = 8;
    const uint64_t cnt = v.size();
    std::memcpy(kv.bytes.data(), &et, 4);
    std::memcpy(kv.bytes.data() + 4, &cnt, 8);
    for (const std::string& s : v) {
        const uint64_t l = s.size();
        const size_t o = kv.bytes.size();
        kv.bytes.resize(o + 8 + s.size());
        std::memcpy(kv.bytes.data() + o, &l, 8);
        std::memcpy(kv.bytes.data() + o + 8, s.data(), s.size());
    }
    kvs_.push_back(std::move(kv));
}
void GGUFWriter::add_tensor(const std::string& name, const std::vector<uint64_t>& dims, bool is_f16, const void* data,
                            uint64_t bytes) {
    tensors_.push_back(T{name, dims, is_f16 ? VSL_WF_F16 : VSL_WF_F32, data, bytes});
}
void GGUFWriter::add_tensor_format(const std::string& name, const std::vector<uint64_t>& dims, int fmt,
                                   const void* data, uint64_t bytes) {
    tensors_.push_back(T{name, dims, fmt, data, bytes});
}

ExpectedVoid GGUFWriter::write(const Path& path) const {
    const uint64_t kAlign = 32;
    std::vector<KV> kvs = kvs_;
    kvs.push_back(KV{"vsl.tensor_type_convention", 8, {}});
    {
        std::string c = conv_ == GGUFConvention::GGML ? "ggml" : "reference";
        uint64_t l = c.size();
        kvs.back().bytes.resize(8 + c.size());
        std::memcpy(kvs.back().bytes.data(), &l, 8);
        std::memcpy(kvs.back().bytes.data() + 8, c.data(), c.size());
    }
    if (conv_ == GGUFConvention::GGML) {
        KV a{"general.alignment", 4, std::vector<uint8_t>(4)};
        uint32_t v = static_cast<uint32_t>(kAlign);
        std::memcpy(a.bytes.data(), &v, 4);
        kvs.push_back(std::move(a));
    }
    // "vsl.pad": a string sized so that the tensor infos end on a 32-byte boundary, making the
    // reference's data-start rule (no padding) and ggml's (align up) agree.
    kvs.push_back(KV{"vsl.pad", 8, std::vector<uint8_t>(8)});
    auto header_bytes = [&]() {
        uint64_t n = 24;
        for (auto& kv : kvs) n += 8 + kv.key.size() + 4 + kv.bytes.size();
        for (auto& t : tensors_) n += 8 + t.name.size() + 4 + 8 * t.dims.size() + 4 + 8;
        return n;
    };
    const uint64_t pad = (kAlign - header_bytes() % kAlign) % kAlign;
    {
        KV& p = kvs.back();
        p.bytes.assign(8 + pad, static_cast<uint8_t>(' '));
        std::memcpy(p.bytes.data(), &pad, 8);
    }
    std::ofstream f(path.string(), std::ios::binary);
    if (!f) return kErrOpen;
    auto put = [&](const void* p, size_t n) { f.write(static_cast<const char*>(p), static_cast<std::streamsize>(n)); };
    uint32_t magic = 0x46554747u, version = 3;
    uint64_t nt = tensors_.size(), nkv = kvs.size();
    put(&magic, 4); put(&version, 4); put(&nt, 8); put(&nkv, 8);
    for (auto& kv : kvs) {
        uint64_t l = kv.key.size();
        put(&l, 8); put(kv.key.data(), kv.key.size()); put(&kv.type, 4); put(kv.bytes.data(), kv.bytes.size());
    }
    uint64_t off = 0;
    std::vector<uint64_t> offs;
    for (auto& t : tensors_) {
        uint64_t l = t.name.size();
        put(&l, 8); put(t.name.data(), t.name.size());
        uint32_t nd = static_cast<uint32_t>(t.dims.size());
        put(&nd, 4);
        for (auto d : t.dims) put(&d, 8);
        // type ids per format F32, F16, Q4_0, Q4_1, Q8_0
        static const uint32_t kRefIds[5] = {6, 48, 13, 14, 17}, kGgmlIds[5] = {0, 1, 2, 3, 8};
        const uint32_t ty = (conv_ == GGUFConvention::GGML ? kGgmlIds : kRefIds)[t.fmt];
        put(&ty, 4);
        put(&off, 8);
        offs.push_back(off);
        off = GGUFLoader::align_offset(off + t.bytes, kAlign);
    }
    static const char zeros[64] = {0};
    uint64_t written = 0;
    for (size_t i = 0; i < tensors_.size(); ++i) {
        if (offs[i] > written) put(zeros, offs[i] - written);
        put(tensors_[i].data, tensors_[i].bytes);
        written = offs[i] + tensors_[i].bytes;
    }
    if (!f) return kErrRead;
    return ExpectedVoid();
}

}  // namespace vk_symbiote
