// Tokenizer.cpp -- vocabulary from GGUF metadata; the reference's whitespace-split encode with
// per-character and hash fallbacks, and its space-joined decode.
#include "Tokenizer.h"

#include <cstring>
#include <sstream>

#include "GGUFLoader.h"

namespace vk_symbiote {

namespace {

constexpr uint32_t kGgufString = 8;
constexpr uint32_t kMaxKeyedId = 100000;  // Tokenizer.cpp:66

// Strings of a metadata array of strings (raw layout: elem type u32, count u64, then (len u64, bytes)*).
bool string_array(const GGUFMetadataKV& kv, std::vector<std::string>& out) {
    const std::vector<uint8_t>& r = kv.raw_value;
    if (kv.value_type != GGUFValueType::ARRAY || r.size() < 12) return false;
    uint32_t et;
    uint64_t cnt;
    std::memcpy(&et, r.data(), 4);
    std::memcpy(&cnt, r.data() + 4, 8);
    if (et != kGgufString) return false;
    size_t o = 12;
    out.clear();
    out.reserve(static_cast<size_t>(std::min<uint64_t>(cnt, r.size() / 8)));
    for (uint64_t i = 0; i < cnt; ++i) {
        uint64_t len;
        if (r.size() - o < 8) return false;
        std::memcpy(&len, r.data() + o, 8);
        o += 8;
        if (r.size() - o < len) return false;
        out.emplace_back(reinterpret_cast<const char*>(r.data() + o), static_cast<size_t>(len));
        o += static_cast<size_t>(len);
    }
    return true;
}

}  // namespace

std::unique_ptr<Tokenizer> Tokenizer::create_simple_tokenizer() {  // Tokenizer.cpp:113-129
    auto t = std::make_unique<Tokenizer>();
    t->vocab_.resize(256);
    for (uint32_t i = 0; i < 256; ++i) {
        t->vocab_[i] = std::string(1, static_cast<char>(i));
        t->token_to_id_map_[t->vocab_[i]] = i;
    }
    t->source_ = Source::BYTES;
    return t;
}

std::unique_ptr<Tokenizer> Tokenizer::from_tokens(const std::vector<std::string>& tokens) {
    if (tokens.empty()) return create_simple_tokenizer();
    auto t = std::make_unique<Tokenizer>();
    t->vocab_ = tokens;
    for (uint32_t i = 0; i < tokens.size(); ++i) t->token_to_id_map_[tokens[i]] = i;  // a repeat: last id wins
    t->source_ = Source::GGUF_ARRAY;
    return t;
}

std::unique_ptr<Tokenizer> Tokenizer::from_gguf(const Path& gguf_path) {
    GGUFLoader g(gguf_path);
    if (!g.load().has_value()) return create_simple_tokenizer();  // unreadable file: byte fallback (:16-27)
    if (const GGUFMetadataKV* kv = g.get_metadata("tokenizer.ggml.tokens")) {
        std::vector<std::string> toks;
        if (string_array(*kv, toks) && !toks.empty()) return from_tokens(toks);
    }
    // string keys "tokenizer.ggml.tokens.<id>" in file order (:48-74)
    auto t = std::make_unique<Tokenizer>();
    for (const std::string& key : g.get_metadata_keys()) {
        if (key.find("tokenizer.ggml") == std::string::npos || key.find("tokens") == std::string::npos) continue;
        const GGUFMetadataKV* kv = g.get_metadata(key);
        if (!kv || static_cast<uint32_t>(kv->value_type) != kGgufString) continue;
        const size_t dot = key.find_last_of('.');
        uint32_t id;
        try {
            id = static_cast<uint32_t>(std::stoul(key.substr(dot + 1)));
        } catch (...) {
            continue;
        }
        if (id >= kMaxKeyedId) continue;
        const std::string value = kv->get_string();
        t->token_to_id_map_[value] = id;
        t->vocab_.resize(id + 1);  // may shrink the list, as the reference's does (:68)
        t->vocab_[id] = value;
    }
    if (t->token_to_id_map_.empty()) return create_simple_tokenizer();
    t->source_ = Source::GGUF_KEYS;
    return t;
}

std::vector<uint32_t> Tokenizer::encode(const std::string& text) const {  // Tokenizer.cpp:131-178
    std::vector<uint32_t> ids;
    std::istringstream iss(text);
    std::string word;
    if (!token_to_id_map_.empty()) {
        while (iss >> word) {
            auto it = token_to_id_map_.find(word);
            if (it != token_to_id_map_.end()) {
                ids.push_back(it->second);
                continue;
            }
            for (char c : word) {
                auto ci = token_to_id_map_.find(std::string(1, c));
                if (ci != token_to_id_map_.end()) {
                    ids.push_back(ci->second);
                } else {
                    // the char is widened with its sign (x86 char is signed), as the reference does
                    const uint32_t h = static_cast<uint32_t>(static_cast<int32_t>(static_cast<signed char>(c))) * 31u;
                    ids.push_back(h % 31000u + 1000u);
                }
            }
        }
    } else {  // no vocabulary: one hashed id per word (:158-170)
        while (iss >> word) {
            uint32_t h = 0;
            for (char c : word) h = h * 31u + static_cast<unsigned char>(c);
            ids.push_back(h % 31000u + 1000u);
        }
    }
    if (ids.empty()) ids.push_back(0);
    return ids;
}

std::string Tokenizer::decode(const std::vector<uint32_t>& tokens) const {  // Tokenizer.cpp:180-198
    std::string r;
    if (vocab_.empty()) return r;
    for (size_t i = 0; i < tokens.size(); ++i) {
        r += vocab_[tokens[i] % vocab_.size()];
        if (i + 1 < tokens.size()) r += ' ';
    }
    return r;
}

uint32_t Tokenizer::vocab_size() const { return static_cast<uint32_t>(vocab_.size()); }

}  // namespace vk_symbiote
