// GGUFLoader's public API as a C++ caller of the reference's header sees it (GGUFLoader.h:265-333):
// compiled against vk_symbiote/GGUFLoader.h and linked with libvsl_engine.so by
// tests/test_cpp_api.py.  Host only: nothing here touches a GPU.
//
// Usage: gguf_api_check <scratch dir>.  Prints one line per check; exits 1 on the first failure.
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <vector>

#include "GGUFLoader.h"

using namespace vk_symbiote;

static int g_checks = 0;
#define CHECK(cond)                                                                  \
    do {                                                                             \
        ++g_checks;                                                                  \
        if (!(cond)) {                                                               \
            std::fprintf(stderr, "FAILED line %d: %s\n", __LINE__, #cond);           \
            std::exit(1);                                                            \
        }                                                                            \
    } while (0)

static std::vector<float> ramp(size_t n, float base) {
    std::vector<float> v(n);
    for (size_t i = 0; i < n; ++i) v[i] = base + 0.5f * static_cast<float>(i);
    return v;
}

int main(int argc, char** argv) {
    if (argc < 2) return 2;
    const std::string dir = argv[1];
    const std::vector<float> a = ramp(64, 1.0f), b = ramp(32, -3.0f), c = ramp(128, 7.0f), b2 = ramp(32, 100.0f);

    // main file: tensors a, b and a vocabulary with scores, token types and tokenizer keys
    {
        GGUFWriter w(GGUFConvention::REFERENCE);
        w.add_u32("llama.embedding_length", 64);
        w.add_string("tokenizer.ggml.model", "llama");
        w.add_u32("tokenizer.ggml.bos_token_id", 1);
        w.add_u32("tokenizer.ggml.eos_token_id", 2);
        w.add_bool("tokenizer.ggml.add_bos_token", true);
        w.add_string("tokenizer.chat_template", "{{x}}");
        w.add_string_array("tokenizer.ggml.tokens", {"<unk>", "<s>", "</s>", std::string("a\0b", 3)});
        const float scores[4] = {0.0f, -1.5f, -2.5f, 3.25f};
        w.add_array("tokenizer.ggml.scores", 6, 4, scores, sizeof(scores));
        const int32_t types[4] = {2, 3, 3, 1};
        w.add_array("tokenizer.ggml.token_type", 5, 4, types, sizeof(types));
        w.add_tensor("t.a", {64}, false, a.data(), a.size() * 4);
        w.add_tensor("t.b", {32}, false, b.data(), b.size() * 4);
        CHECK(w.write(dir + "/main.gguf").has_value());
    }
    // shard in the other tensor-type convention: c, plus a second "t.b" that the main file shadows
    {
        GGUFWriter w(GGUFConvention::GGML);
        w.add_tensor("t.c", {128}, false, c.data(), c.size() * 4);
        w.add_tensor("t.b", {32}, false, b2.data(), b2.size() * 4);
        CHECK(w.write(dir + "/shard.gguf").has_value());
    }

    GGUFLoader g(dir + "/main.gguf");
    CHECK(!g.add_shard(dir + "/shard.gguf").has_value());  // not loaded yet
    CHECK(g.load().has_value());
    CHECK(g.is_valid() && g.get_version() == 3);

    // vocabulary and tokenizer configuration
    const auto& voc = g.get_vocabulary();
    CHECK(voc.size() == 4);
    CHECK(voc[1].token == "<s>" && voc[3].bytes.size() == 3 && voc[3].bytes[1] == 0);
    CHECK(voc[3].score == 3.25f && voc[1].score == -1.5f);
    CHECK(voc[0].token_type == 2 && voc[3].token_type == 1);
    const TokenizerConfig& tc = g.get_tokenizer_config();
    CHECK(tc.model_type == "llama" && tc.bos_token_id == 1 && tc.eos_token_id == 2);
    CHECK(tc.add_bos_token && !tc.add_eos_token && tc.chat_template == "{{x}}");
    std::printf("vocabulary ok\n");

    // metadata arrays (GGUFMetadataKV, GGUFLoader.h:95-104): the element type, and the element bytes
    // without the u32 type + u64 count header
    const GGUFMetadataKV* sc = g.get_metadata("tokenizer.ggml.scores");
    CHECK(sc != nullptr && sc->value_type == GGUFValueType::ARRAY);
    CHECK(sc->get_array_element_type() == GGUFValueType::FLOAT32);
    const std::vector<uint8_t> sb = sc->get_array_data();
    const float want_scores[4] = {0.0f, -1.5f, -2.5f, 3.25f};
    CHECK(sb.size() == sizeof(want_scores) && std::memcmp(sb.data(), want_scores, sizeof(want_scores)) == 0);
    const GGUFMetadataKV* ty = g.get_metadata("tokenizer.ggml.token_type");
    CHECK(ty != nullptr && ty->get_array_element_type() == GGUFValueType::INT32);
    const std::vector<uint8_t> tb = ty->get_array_data();
    int32_t t3 = 0;
    CHECK(tb.size() == 16);
    std::memcpy(&t3, tb.data() + 12, 4);
    CHECK(t3 == 1);
    const GGUFMetadataKV* tk = g.get_metadata("tokenizer.ggml.tokens");
    CHECK(tk != nullptr && tk->get_array_element_type() == GGUFValueType::STRING);
    CHECK(tk->get_array_data().size() == 4 * 8 + 5 + 3 + 4 + 3);  // (u64 length, bytes) per string
    const GGUFMetadataKV* bos = g.get_metadata("tokenizer.ggml.bos_token_id");
    CHECK(bos != nullptr && bos->get_array_element_type() == GGUFValueType::UINT8 && bos->get_array_data().empty());
    // every tensor-type id of the reference's enum is declared
    static_assert(static_cast<uint32>(GGUFValueType::Q8_1) == 18 && static_cast<uint32>(GGUFValueType::Q6_K) == 23 &&
                      static_cast<uint32>(GGUFValueType::IQ4_NL) == 31 && static_cast<uint32>(GGUFValueType::IQ4_XS_2) == 46 &&
                      static_cast<uint32>(GGUFValueType::IQ2_M) == 49 && static_cast<uint32>(GGUFValueType::IQ4_XS_3) == 53,
                  "GGUFValueType ids");
    std::printf("metadata arrays ok\n");

    // shards
    CHECK(!g.is_sharded());
    CHECK(g.get_tensor("t.c") == nullptr);
    CHECK(g.add_shard(dir + "/shard.gguf").has_value());
    CHECK(g.add_shard(dir + "/missing.gguf").error() == -1);
    CHECK(g.is_sharded());
    CHECK(g.tensor_count() == 4);
    const auto names = g.get_tensor_names();
    CHECK((names == std::vector<std::string>{"t.a", "t.b", "t.c"}));
    const GGUFTensorInfo* tcinfo = g.get_tensor("t.c");
    CHECK(tcinfo != nullptr);
    auto rc = g.read_tensor_data(*tcinfo);
    CHECK(rc.has_value() && rc.value() == c);
    auto rb = g.read_tensor_data(*g.get_tensor("t.b"));
    CHECK(rb.has_value() && rb.value() == b);  // the main file's t.b
    CHECK(g.generate_packs(g.get_model_config()).size() == 3);
    std::printf("shards ok\n");

    // stream_tensors_parallel: one result per name, in order
    auto st = g.stream_tensors_parallel({"t.c", "nope", "t.a", "t.b"}, 3);
    CHECK(st.size() == 4);
    CHECK(st[0].has_value() && st[0].value() == c);
    CHECK(!st[1].has_value() && st[1].error() == -30);
    CHECK(st[2].has_value() && st[2].value() == a);
    CHECK(st[3].has_value() && st[3].value() == b);
    CHECK(g.stream_tensors_parallel({}, 4).empty());
    std::printf("stream ok\n");

    // cache: two entries at most
    TensorCacheConfig cfg;
    cfg.max_entries = 2;
    g.configure_cache(cfg);
    CHECK(g.get_tensor_cache_size() == 0);
    CHECK(g.read_tensor_cached("t.a").value() == a);  // miss
    CHECK(g.read_tensor_cached("t.a").value() == a);  // hit
    CHECK(g.read_tensor_cached("t.b").value() == b);  // miss
    CHECK(g.get_tensor_cache_size() == (64 + 32) * 4);
    CHECK(g.read_tensor_cached("t.c").value() == c);  // miss, evicts t.a (least recently used)
    TensorLRUCache::Stats s = g.get_cache_stats();
    CHECK(s.hits == 1 && s.misses == 3 && s.evictions == 1 && s.current_entries == 2);
    CHECK(s.current_memory_bytes == (32 + 128) * 4);
    CHECK(std::fabs(s.hit_rate() - 0.25) < 1e-12);
    CHECK(g.read_tensor_cached("zzz").error() == -30);
    g.clear_tensor_cache();
    CHECK(g.get_tensor_cache_size() == 0 && g.get_cache_stats().current_entries == 0);
    cfg.max_memory_bytes = 100;  // smaller than any tensor here: nothing is kept
    g.configure_cache(cfg);
    CHECK(g.read_tensor_cached("t.a").value() == a);
    CHECK(g.get_tensor_cache_size() == 0);
    std::printf("cache ok\n");

    // Expected<T>: value / error states, copies and moves
    Expected<std::vector<float>> e1(a), e2(-20);
    CHECK(e1.has_value() && static_cast<bool>(e1) && e1.error() == 0 && e1.value() == a);
    CHECK(!e2.has_value() && !static_cast<bool>(e2) && e2.error() == -20);
    bool threw = false;
    try {
        (void)e2.value();
    } catch (const std::runtime_error&) {
        threw = true;
    }
    CHECK(threw);
    Expected<std::vector<float>> e3 = e1, e4 = std::move(e2);
    CHECK(e3.value() == a && e4.error() == -20);
    e3 = e4;
    CHECK(!e3.has_value() && e3.error() == -20);
    ExpectedVoid v0, v1(-3), v2(0);
    CHECK(v0.has_value() && v0.error() == 0 && !v1.has_value() && v1.error() == -3 && !v2.has_value());
    std::printf("expected ok\n");

    CHECK(g.close().has_value());
    CHECK(!g.is_sharded() && g.get_vocabulary().empty());
    std::printf("all %d checks passed\n", g_checks);
    return 0;
}
