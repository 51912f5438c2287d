// Common.h -- shared types of the MI355X backend, kept source-compatible with the reference's
// vk_symbiote/include/vk_symbiote/Common.h (ModelConfig :56-76, InferenceParams :78-86,
// Expected<T> :88-193, Path :195-202, PerformanceMetrics :285-318) minus the Vulkan includes.
#pragma once

#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstddef>
#include <cstdint>
#include <filesystem>
#include <new>
#include <optional>
#include <stdexcept>
#include <string>
#include <utility>
#include <variant>
#include <vector>

namespace vk_symbiote {

using uint8 = uint8_t;
using uint32 = uint32_t;
using uint64 = uint64_t;
using int8 = int8_t;
using int32 = int32_t;
using int64 = int64_t;
using float16 = uint16_t;

struct ModelConfig {
    uint32 hidden_size = 4096;
    uint32 num_layers = 32;
    uint32 num_attention_heads = 32;
    uint32 num_key_value_heads = 32;
    uint32 intermediate_size = 11008;
    uint32 vocab_size = 32000;
    float rope_theta = 10000.0f;
    uint32 max_position_embeddings = 2048;
    std::string model_type = "llama";
    uint32 head_dim = 128;
    bool use_fp16 = true;
    float rms_epsilon = 1e-5f;

    // Windowed long-context mode of the reference (Common.h:70-75).  The engine sets these from
    // EngineOptions (off unless asked for); sparse_threshold is the reference's fixed
    // `seq_len > 8192` switch (VulkanSymbioteEngine.cpp:788).  sparse_block_size and
    // use_ring_attention are kept for API compatibility (the reference never reads them).
    bool use_sparse_attention = true;
    uint32 sparse_window_size = 512;
    uint32 sparse_global_tokens = 16;
    uint32 sparse_block_size = 1024;
    bool use_ring_attention = true;
    uint32 sparse_threshold = 8192;
};

struct InferenceParams {
    uint32 max_new_tokens = 256;
    float temperature = 0.7f;
    float top_p = 0.9f;
    uint32 top_k = 40;
    bool do_sample = true;
    float repetition_penalty = 1.1f;
    uint32 context_length = 2048;
};

// A value or an integer error code: the public interface of the reference's Expected<T>
// (Common.h:88-193) -- construction from a value or from an int code, has_value(), explicit bool,
// value() (throws std::runtime_error on an error) and error() (0 while a value is held).  Stored as
// a std::variant of the value and a tagged code, so copies, moves and destruction are the variant's.
template <typename T>
class Expected {
    struct Failure {
        int code;
    };
    std::variant<T, Failure> state_;

    [[noreturn]] void fail_access() const {
        throw std::runtime_error("Expected::value() called on error state (code " + std::to_string(error()) + ")");
    }

   public:
    Expected() : state_(std::in_place_index<0>) {}
    Expected(const T& val) : state_(std::in_place_index<0>, val) {}
    Expected(T&& val) : state_(std::in_place_index<0>, std::move(val)) {}
    Expected(int err) : state_(std::in_place_index<1>, Failure{err}) {}

    bool has_value() const noexcept { return state_.index() == 0; }
    explicit operator bool() const noexcept { return has_value(); }
    T& value() {
        if (T* p = std::get_if<0>(&state_)) return *p;
        fail_access();
    }
    const T& value() const {
        if (const T* p = std::get_if<0>(&state_)) return *p;
        fail_access();
    }
    int error() const noexcept {
        const Failure* f = std::get_if<1>(&state_);
        return f ? f->code : 0;
    }
};

// Success, or the error code it was constructed with (any int, 0 included, means failure).
template <>
class Expected<void> {
    std::optional<int> failure_;

   public:
    Expected() = default;
    Expected(int err) : failure_(err) {}
    bool has_value() const noexcept { return !failure_.has_value(); }
    explicit operator bool() const noexcept { return has_value(); }
    int error() const noexcept { return failure_.value_or(0); }
};
using ExpectedVoid = Expected<void>;

inline ExpectedVoid make_expected_success() { return ExpectedVoid(); }

struct Path : public std::filesystem::path {
    Path() : std::filesystem::path() {}
    Path(const std::string& p) : std::filesystem::path(p) {}
    Path(const char* p) : std::filesystem::path(p) {}
    Path(const std::filesystem::path& p) : std::filesystem::path(p) {}
    const char* c_str() const noexcept { return native().c_str(); }
};

inline uint64 get_current_time_ns() {
    return std::chrono::duration_cast<std::chrono::nanoseconds>(
               std::chrono::high_resolution_clock::now().time_since_epoch())
        .count();
}

inline float silu(float x) { return x / (1.0f + std::exp(-x)); }

// Performance monitoring (Common.h:285-318).  update() here takes the decode wall time of a whole
// generation and the number of tokens it produced, so average_tokens_per_second is a rate.
struct PerformanceMetrics {
    uint64_t total_inference_time_ns = 0;
    uint64_t total_gpu_time_ns = 0;
    uint64_t total_cpu_time_ns = 0;
    uint32_t total_inferences = 0;
    uint32_t successful_inferences = 0;
    float average_tokens_per_second = 0.0f;
    float gpu_utilization_percent = 0.0f;
    float memory_bandwidth_gbps = 0.0f;

    void reset() { *this = PerformanceMetrics(); }
    void update(uint64_t inference_time_ns, uint32_t tokens_generated) {
        total_inferences++;
        if (inference_time_ns > 0) {
            total_inference_time_ns += inference_time_ns;
            successful_inferences++;
            if (tokens_generated > 0)
                average_tokens_per_second =
                    static_cast<float>(tokens_generated) / (static_cast<float>(inference_time_ns) / 1e9f);
        }
    }
};

// Error codes carried by Expected<T> (negative ints, as the reference's loader codes).
enum ErrorCode : int {
    kErrOpen = -1,
    kErrMagic = -2,
    kErrMetadata = -3,
    kErrTensorInfo = -4,
    kErrCapacity = -5,
    kErrRead = -11,
    kErrUnsupportedType = -12,
    kErrUnsupportedQuant = -20,
    kErrNotFound = -30,
    kErrDevice = -50,
    kErrInvalid = -60,
};

}  // namespace vk_symbiote
