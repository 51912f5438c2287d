// NomadPack.cpp -- pack metadata helpers and the resident-pack registry.
#include "NomadPack.h"

#include <cstdlib>
#include <string>

namespace vk_symbiote {

// PackMetadata::type by tensor name, in the reference's order (GGUFLoader.cpp:1302-1315): ffn_up is
// filed under FEED_FORWARD_GATE and only attn_norm / ffn_norm are NORM_GAMMA, so output_norm falls
// through to HEAD ("output").
PackType classify_tensor_type(const std::string& name) {
    auto has = [&](const char* s) { return name.find(s) != std::string::npos; };
    if (has("attn_q")) return PackType::ATTENTION_Q;
    if (has("attn_k")) return PackType::ATTENTION_K;
    if (has("attn_v")) return PackType::ATTENTION_V;
    if (has("attn_o") || has("attn_output")) return PackType::ATTENTION_O;
    if (has("ffn_gate") || has("ffn_up")) return PackType::FEED_FORWARD_GATE;
    if (has("ffn_down")) return PackType::FEED_FORWARD_DOWN;
    if (has("ffn_norm") || has("attn_norm")) return PackType::NORM_GAMMA;
    if (has("token_embd")) return PackType::EMBEDDING;
    if (has("output")) return PackType::HEAD;
    return PackType::UNKNOWN;
}

// The first "blk.<digits>" anywhere in the name -> the digits (GGUFLoader.cpp:1264-1272, a regex
// search for blk\.(\d+) and std::stoul), 0 when there is none.  A value past 2^64 - 1 (where the
// reference's stoul throws) reads as 0; otherwise the value is truncated to 32 bits as the
// reference's return type does.
uint32 extract_layer_index(const std::string& name) {
    for (size_t at = name.find("blk."); at != std::string::npos; at = name.find("blk.", at + 1)) {
        const size_t d0 = at + 4;
        size_t d1 = d0;
        while (d1 < name.size() && name[d1] >= '0' && name[d1] <= '9') ++d1;
        if (d1 == d0) continue;
        try {
            return static_cast<uint32>(std::stoul(name.substr(d0, d1 - d0)));
        } catch (...) {
            return 0;
        }
    }
    return 0;
}

// GGUFLoader.cpp:1279-1300: 0.5 base, +0.2 attention, +0.3 embedding/output, +0.1 first four layers.
float calculate_pack_priority(const std::string& name) {
    float p = 0.5f;
    if (name.find("attn") != std::string::npos) p += 0.2f;
    if (name.find("token_embd") != std::string::npos || name.find("output") != std::string::npos) p += 0.3f;
    if (extract_layer_index(name) < 4) p += 0.1f;
    return p < 1.0f ? p : 1.0f;
}

void PackManager::register_pack(const PackMetadata& meta, void* device_ptr, uint64 bytes, int dtype) {
    auto it = index_.find(meta.tensor_name);
    ResidentPack rp{meta, device_ptr, bytes, dtype, MemoryTier::VRAM_HOT};
    if (it != index_.end()) {
        packs_[it->second] = rp;
        return;
    }
    index_[meta.tensor_name] = packs_.size();
    packs_.push_back(rp);
}

const ResidentPack* PackManager::find(const std::string& tensor_name) const {
    auto it = index_.find(tensor_name);
    return it == index_.end() ? nullptr : &packs_[it->second];
}

uint64 PackManager::resident_bytes() const {
    uint64 n = 0;
    for (auto& p : packs_) n += p.bytes;
    return n;
}

}  // namespace vk_symbiote
