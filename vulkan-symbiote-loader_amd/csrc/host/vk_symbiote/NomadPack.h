// NomadPack.h -- pack metadata and the HBM-resident pack manager.
//
// Keeps the reference's pack granularity and metadata (PackType / MemoryTier / PackMetadata /
// MemoryPoolStats, vk_symbiote/include/vk_symbiote/NomadPack.h:26-57; one pack per GGUF tensor,
// pack_id = std::hash(name), priority rules GGUFLoader.cpp:730-751, 1279-1300).  On MI355X every
// pack is uploaded once (pinned host staging -> hipMemcpyAsync on a side stream) into one HBM
// arena and stays resident: 288 GB of HBM holds any model this backend serves, so the reference's
// VRAM/RAM/disk tiers, eviction and defragmentation have no work to do.
#pragma once

#include <cstdint>
#include <string>
#include <unordered_map>
#include <vector>

#include "Common.h"

struct vsl_arena;

namespace vk_symbiote {

enum class PackType : uint8 {
    ATTENTION_Q = 0, ATTENTION_K = 1, ATTENTION_V = 2, ATTENTION_O = 3,
    FEED_FORWARD_GATE = 4, FEED_FORWARD_UP = 5, FEED_FORWARD_DOWN = 6,
    NORM_GAMMA = 7, NORM_BETA = 8, ROPE = 9, EMBEDDING = 10, HEAD = 11, UNKNOWN = 255
};

enum class MemoryTier : uint8 { VRAM_HOT = 0, RAM_WARM = 1, DISK_COLD = 2, UNLOADED = 3 };

struct PackMetadata {
    uint64 pack_id = 0;
    PackType type = PackType::UNKNOWN;
    uint32 layer_idx = 0, head_idx = 0, head_group_idx = 0;
    size_t compressed_size = 0, decompressed_size = 0;
    uint64 file_offset = 0;
    std::string tensor_name;
    float base_priority = 0.5f;
    uint32 alignment = 256;
    uint32 n_dimensions = 0;
    std::vector<uint64_t> dimensions;
};

struct MemoryPoolStats {
    uint64 total_size = 0, used_size = 0, free_size = 0;
    uint32 allocation_count = 0;
    float fragmentation_ratio = 0.0f;
};

PackType classify_tensor_type(const std::string& name);
uint32 extract_layer_index(const std::string& name);
float calculate_pack_priority(const std::string& name);

// A resident pack: metadata + where it lives in HBM.
struct ResidentPack {
    PackMetadata meta;
    void* device_ptr = nullptr;
    uint64 bytes = 0;
    int dtype = 0;  // VSL_DT_*
    MemoryTier tier = MemoryTier::UNLOADED;
};

class PackManager {
   public:
    PackManager() = default;
    void register_pack(const PackMetadata& meta, void* device_ptr, uint64 bytes, int dtype);
    const ResidentPack* find(const std::string& tensor_name) const;
    const std::vector<ResidentPack>& packs() const { return packs_; }
    uint64 resident_bytes() const;
    void clear() {
        packs_.clear();
        index_.clear();
    }

   private:
    std::vector<ResidentPack> packs_;
    std::unordered_map<std::string, size_t> index_;
};

}  // namespace vk_symbiote
