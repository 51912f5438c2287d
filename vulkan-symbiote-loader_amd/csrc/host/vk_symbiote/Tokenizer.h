// Tokenizer.h -- the reference's Tokenizer API (vk_symbiote/include/vk_symbiote/Tokenizer.h:7-22):
// from_gguf / encode / decode / vocab_size, with the reference's encode and decode algorithms
// (vk_symbiote/src/Tokenizer.cpp:131-198) and its 256-byte fallback vocabulary (:113-129).
//
// from_gguf reads the vocabulary through GGUFLoader instead of the reference's own scan, which reads
// the value type before the key (Tokenizer.cpp:41-46) and so never parses a real file.  Sources, in
// order: the standard string array "tokenizer.ggml.tokens" (id = array index), then string keys
// "tokenizer.ggml.tokens.<id>" as the reference's scan meant to read them (:55-74: id parsed by
// std::stoul after the last '.', kept below 100000, the list resized to id + 1 at every key), then
// the byte fallback.
#pragma once

#include <cstdint>
#include <memory>
#include <string>
#include <unordered_map>
#include <vector>

#include "Common.h"

namespace vk_symbiote {

class Tokenizer {
   public:
    enum class Source { BYTES = 0, GGUF_ARRAY = 1, GGUF_KEYS = 2 };

    static std::unique_ptr<Tokenizer> from_gguf(const Path& gguf_path);
    static std::unique_ptr<Tokenizer> create_simple_tokenizer();
    // additive: a vocabulary given as a list (id = index)
    static std::unique_ptr<Tokenizer> from_tokens(const std::vector<std::string>& tokens);

    std::vector<uint32_t> encode(const std::string& text) const;
    std::string decode(const std::vector<uint32_t>& tokens) const;
    uint32_t vocab_size() const;
    Source source() const { return source_; }

   private:
    std::vector<std::string> vocab_;
    std::unordered_map<std::string, uint32_t> token_to_id_map_;
    Source source_ = Source::BYTES;
};

}  // namespace vk_symbiote
