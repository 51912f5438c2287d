// NomadPack.cpp -- pack metadata helpers and the resident-pack registry.
#include "NomadPack.h"

#include <cstdlib>

namespace vk_symbiote {

// Tensor-name classification used for PackMetadata::type (the reference's classify_tensor_type).
PackType classify_tensor_type(const std::string& name) {
    auto has = [&](const char* s) { return name.find(s) != std::string::npos; };
    if (has("attn_q")) return PackType::ATTENTION_Q;
    if (has("attn_k")) return PackType::ATTENTION_K;
    if (has("attn_v")) return PackType::ATTENTION_V;
    if (has("attn_o") || has("attn_output")) return PackType::ATTENTION_O;
    if (has("ffn_gate")) return PackType::FEED_FORWARD_GATE;
    if (has("ffn_up")) return PackType::FEED_FORWARD_UP;
    if (has("ffn_down")) return PackType::FEED_FORWARD_DOWN;
    if (has("norm")) return PackType::NORM_GAMMA;
    if (has("token_embd")) return PackType::EMBEDDING;
    if (has("output")) return PackType::HEAD;
    return PackType::UNKNOWN;
}

// "blk.<n>." prefix -> n (GGUFLoader.cpp:1264-1272), 0 otherwise.
uint32 extract_layer_index(const std::string& name) {
    if (name.compare(0, 4, "blk.") != 0) return 0;
    const char* p = name.c_str() + 4;
    char* end = nullptr;
    unsigned long v = std::strtoul(p, &end, 10);
    return end == p ? 0u : static_cast<uint32>(v);
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
