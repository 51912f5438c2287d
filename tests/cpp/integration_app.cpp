// The C++ drop-in program a reference application would be (basic_inference.cpp:25-32 and
// examples/benchmark.cpp:137-170 use the same calls): ConfigManager from the command line, the
// engine from the model path, generate() and run_benchmark().  Compiled against
// vk_symbiote/*.h + libvsl_engine.so by tests/test_cpp_api.py (CPU) and run on a GPU by
// tests/test_engine_gpu.py.
//
// Usage: integration_app --model <file.gguf> [--kv-capacity N] <prompt>
// Prints "generate: <text>" and "benchmark: <avg tok/s> <min> <max>".
#include <cstdio>
#include <exception>
#include <string>

#include "ConfigManager.h"
#include "VulkanSymbioteEngine.h"

int main(int argc, char** argv) {
    try {
        vk_symbiote::ConfigManager::instance().load_from_args(argc, argv);
        vk_symbiote::VulkanSymbioteEngine engine(vk_symbiote::ConfigManager::instance().model_path());
        const std::string prompt = argc > 1 ? argv[argc - 1] : "hello world";
        std::string out = engine.generate(prompt, 8, 0.0f);  // VulkanSymbioteEngine.h:86
        std::printf("generate: ");
        std::fwrite(out.data(), 1, out.size(), stdout);  // any byte, NUL included
        std::printf("\n");
        auto r = engine.run_benchmark(2, 8, 2);  // :98
        std::printf("benchmark: %.3f %.3f %.3f\n", r.avg_tokens_per_sec, r.min_tokens_per_sec, r.max_tokens_per_sec);
        return 0;
    } catch (const std::exception& e) {
        std::fprintf(stderr, "error: %s\n", e.what());
        return 1;
    }
}
