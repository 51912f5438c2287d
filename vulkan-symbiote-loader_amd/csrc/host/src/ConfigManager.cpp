// ConfigManager.cpp -- line-based TOML subset (vk_symbiote/src/ConfigManager.cpp:27-120 parser
// rules: '#' comments, [section], key = value with bool / integer / float / quoted string),
// section mapping (:300-660), CLI (:669-689 plus this backend's flags) and validation (:770-790).
#include "ConfigManager.h"

#include <chrono>
#include <ctime>
#include <fstream>
#include <iomanip>
#include <iostream>
#include <sstream>

namespace vk_symbiote {

std::unique_ptr<ConfigManager> ConfigManager::instance_ = nullptr;
std::mutex ConfigManager::instance_mutex_;

ConfigManager& ConfigManager::instance() {
    std::lock_guard<std::mutex> lock(instance_mutex_);
    if (!instance_) {
        instance_ = std::make_unique<ConfigManager>(PrivateTag{});
        instance_->set_defaults();
    }
    return *instance_;
}

static std::string trim(const std::string& s) {
    size_t a = s.find_first_not_of(" \t\r\n");
    if (a == std::string::npos) return "";
    size_t b = s.find_last_not_of(" \t\r\n");
    return s.substr(a, b - a + 1);
}

static ConfigManager::Value parse_value(std::string v) {
    if (v == "true") return true;
    if (v == "false") return false;
    if (!v.empty() && v.find_first_not_of("0123456789-") == std::string::npos) {
        try {
            return static_cast<int64_t>(std::stoll(v));
        } catch (...) {
            return v;
        }
    }
    if (v.find_first_of(".eE") != std::string::npos) {
        try {
            size_t used = 0;
            double d = std::stod(v, &used);
            if (used == v.size()) return d;
        } catch (...) {
        }
    }
    if (v.size() >= 2 && ((v.front() == '"' && v.back() == '"') || (v.front() == '\'' && v.back() == '\'')))
        v = v.substr(1, v.size() - 2);
    return v;
}

bool ConfigManager::load_from_file(const Path& config_path) {
    std::ifstream file(config_path.string());
    if (!file.is_open()) {
        std::cerr << "Warning: Could not open config file: " << config_path << std::endl;
        return false;
    }
    std::string line, section;
    while (std::getline(file, line)) {
        line = trim(line);
        if (line.empty() || line[0] == '#') continue;
        if (line.front() == '[' && line.back() == ']') {
            section = trim(line.substr(1, line.size() - 2));
            continue;
        }
        size_t eq = line.find('=');
        if (eq == std::string::npos || section.empty()) continue;
        std::string key = trim(line.substr(0, eq));
        std::string val = trim(line.substr(eq + 1));
        // strip a trailing comment outside quotes
        if (!val.empty() && val.front() != '"' && val.front() != '\'') {
            size_t h = val.find('#');
            if (h != std::string::npos) val = trim(val.substr(0, h));
        }
        toml_data_[section][key] = parse_value(val);
    }
    apply_document();
    return validate_config();
}

void ConfigManager::apply_document() {
    auto sec = [&](const char* s) -> const std::unordered_map<std::string, Value>* {
        auto it = toml_data_.find(s);
        return it == toml_data_.end() ? nullptr : &it->second;
    };
    auto num = [](const Value& v, double& out) {
        if (std::holds_alternative<int64_t>(v)) { out = static_cast<double>(std::get<int64_t>(v)); return true; }
        if (std::holds_alternative<double>(v)) { out = std::get<double>(v); return true; }
        return false;
    };
    auto set_f = [&](const std::unordered_map<std::string, Value>* t, const char* k, float& dst) {
        if (!t) return;
        auto it = t->find(k);
        double d;
        if (it != t->end() && num(it->second, d)) dst = static_cast<float>(d);
    };
    auto set_u = [&](const std::unordered_map<std::string, Value>* t, const char* k, uint32_t& dst) {
        if (!t) return;
        auto it = t->find(k);
        if (it != t->end() && std::holds_alternative<int64_t>(it->second)) dst = static_cast<uint32_t>(std::get<int64_t>(it->second));
    };
    auto set_b = [&](const std::unordered_map<std::string, Value>* t, const char* k, bool& dst) {
        if (!t) return;
        auto it = t->find(k);
        if (it != t->end() && std::holds_alternative<bool>(it->second)) dst = std::get<bool>(it->second);
    };
    auto set_s = [&](const std::unordered_map<std::string, Value>* t, const char* k, std::string& dst) {
        if (!t) return;
        auto it = t->find(k);
        if (it != t->end() && std::holds_alternative<std::string>(it->second)) dst = std::get<std::string>(it->second);
    };
    if (auto* t = sec("memory")) {
        set_f(t, "vram_budget_gb", memory_config_.vram_budget_gb);
        set_f(t, "ram_budget_gb", memory_config_.ram_budget_gb);
        set_u(t, "prefetch_lookahead", memory_config_.prefetch_lookahead);
        set_f(t, "eviction_aggression", memory_config_.eviction_aggression);
        set_b(t, "enable_compression", memory_config_.enable_compression);
        set_s(t, "compression_algorithm", memory_config_.compression_algorithm);
        set_u(t, "max_packs_in_memory", memory_config_.max_packs_in_memory);
        set_b(t, "enable_defrag", memory_config_.enable_defrag);
        set_u(t, "defrag_interval_ms", memory_config_.defrag_interval_ms);
    }
    if (auto* t = sec("performance")) {
        set_b(t, "enable_gpu", perf_config_.enable_gpu);
        set_b(t, "enable_profiling", perf_config_.enable_profiling);
        set_u(t, "workgroup_size_x", perf_config_.workgroup_size_x);
        set_u(t, "workgroup_size_y", perf_config_.workgroup_size_y);
        set_u(t, "workgroup_size_z", perf_config_.workgroup_size_z);
        set_b(t, "use_subgroup_ops", perf_config_.use_subgroup_ops);
        set_u(t, "subgroup_size", perf_config_.subgroup_size);
        set_b(t, "use_fp16_math", perf_config_.use_fp16_math);
        set_f(t, "scale_factor", perf_config_.scale_factor);
        set_u(t, "thread_pool_size", perf_config_.thread_pool_size);
        set_u(t, "kv_capacity", perf_config_.kv_capacity);
        uint32_t dev = static_cast<uint32_t>(perf_config_.device);
        set_u(t, "device", dev);
        perf_config_.device = static_cast<int>(dev);
    }
    if (auto* t = sec("logging")) {
        uint32_t lvl = static_cast<uint32_t>(logging_config_.log_level);
        set_u(t, "log_level", lvl);
        logging_config_.log_level = static_cast<LogLevel>(lvl);
        set_b(t, "log_to_file", logging_config_.log_to_file);
        set_s(t, "log_file_path", logging_config_.log_file_path);
        set_b(t, "log_performance", logging_config_.log_performance);
        set_b(t, "log_memory_usage", logging_config_.log_memory_usage);
        set_u(t, "max_log_file_size_mb", logging_config_.max_log_file_size_mb);
    }
    if (auto* t = sec("power")) {
        set_b(t, "enable_power_management", power_config_.enable_power_management);
        set_b(t, "enable_power_saver", power_config_.enable_power_saver);
        set_b(t, "auto_detect_battery", power_config_.auto_detect_battery);
        set_u(t, "power_profile", power_config_.power_profile);
        set_f(t, "battery_threshold_low", power_config_.battery_threshold_low);
        set_f(t, "battery_threshold_critical", power_config_.battery_threshold_critical);
    }
    if (auto* t = sec("benchmark")) {
        set_b(t, "enable_benchmark_mode", benchmark_config_.enable_benchmark_mode);
        set_u(t, "warmup_tokens", benchmark_config_.warmup_tokens);
        set_u(t, "benchmark_tokens", benchmark_config_.benchmark_tokens);
        set_u(t, "iterations", benchmark_config_.iterations);
        set_b(t, "output_json", benchmark_config_.output_json);
        set_s(t, "output_file", benchmark_config_.output_file);
    }
    if (auto* t = sec("codec")) {
        set_s(t, "codec", codec_config_.codec);
        set_u(t, "compression_level", codec_config_.compression_level);
    }
    if (auto* t = sec("batch")) {
        set_b(t, "enable_batching", batch_config_.enable_batching);
        set_u(t, "max_batch_size", batch_config_.max_batch_size);
        set_u(t, "max_sequence_length", batch_config_.max_sequence_length);
    }
    if (auto* t = sec("vitality")) {
        set_b(t, "enabled", vitality_config_.enabled);
        set_f(t, "learning_rate", vitality_config_.learning_rate);
    }
    if (auto* t = sec("shader")) {
        set_s(t, "cache_dir", shader_config_.cache_dir);
        set_b(t, "enable_cache", shader_config_.enable_cache);
        set_b(t, "auto_tune", shader_config_.auto_tune);
    }
    if (auto* t = sec("model")) {
        set_s(t, "path", model_path_);
        set_s(t, "type", model_type_);
    }
}

bool ConfigManager::save_to_file(const Path& config_path) { return save_to_toml(config_path); }

bool ConfigManager::save_to_toml(const Path& config_path) {
    std::ofstream f(config_path.string());
    if (!f.is_open()) return false;
    f << std::boolalpha << std::setprecision(9);
    f << "[memory]\n"
      << "vram_budget_gb = " << memory_config_.vram_budget_gb << "\n"
      << "ram_budget_gb = " << memory_config_.ram_budget_gb << "\n"
      << "prefetch_lookahead = " << memory_config_.prefetch_lookahead << "\n"
      << "eviction_aggression = " << memory_config_.eviction_aggression << "\n"
      << "enable_compression = " << memory_config_.enable_compression << "\n"
      << "compression_algorithm = \"" << memory_config_.compression_algorithm << "\"\n\n";
    f << "[performance]\n"
      << "enable_gpu = " << perf_config_.enable_gpu << "\n"
      << "enable_profiling = " << perf_config_.enable_profiling << "\n"
      << "workgroup_size_x = " << perf_config_.workgroup_size_x << "\n"
      << "use_fp16_math = " << perf_config_.use_fp16_math << "\n"
      << "device = " << perf_config_.device << "\n"
      << "kv_capacity = " << perf_config_.kv_capacity << "\n\n";
    f << "[logging]\n"
      << "log_level = " << static_cast<int>(logging_config_.log_level) << "\n"
      << "log_to_file = " << logging_config_.log_to_file << "\n"
      << "log_file_path = \"" << logging_config_.log_file_path << "\"\n\n";
    f << "[power]\n"
      << "power_profile = " << power_config_.power_profile << "\n\n";
    f << "[benchmark]\n"
      << "enable_benchmark_mode = " << benchmark_config_.enable_benchmark_mode << "\n"
      << "warmup_tokens = " << benchmark_config_.warmup_tokens << "\n"
      << "benchmark_tokens = " << benchmark_config_.benchmark_tokens << "\n"
      << "iterations = " << benchmark_config_.iterations << "\n\n";
    f << "[model]\n"
      << "path = \"" << model_path_ << "\"\n"
      << "type = \"" << model_type_ << "\"\n";
    return static_cast<bool>(f);
}

void ConfigManager::load_from_args(int argc, char* argv[]) {
    for (int i = 1; i < argc; ++i) {
        std::string a = argv[i];
        if (a == "--model" && i + 1 < argc) model_path_ = argv[++i];
        else if (a == "--config" && i + 1 < argc) load_from_file(argv[++i]);
        else if (a == "--vram-gb" && i + 1 < argc) memory_config_.vram_budget_gb = std::stof(argv[++i]);
        else if (a == "--ram-gb" && i + 1 < argc) memory_config_.ram_budget_gb = std::stof(argv[++i]);
        else if (a == "--verbose" || a == "-v") logging_config_.log_level = LogLevel::DEBUG;
        else if (a == "--power-profile" && i + 1 < argc) power_config_.power_profile = std::stoul(argv[++i]);
        else if (a == "--benchmark") benchmark_config_.enable_benchmark_mode = true;
        else if (a == "--disable-gpu") perf_config_.enable_gpu = false;
        else if (a == "--device" && i + 1 < argc) perf_config_.device = std::stoi(argv[++i]);
        else if (a == "--seed" && i + 1 < argc) perf_config_.seed = std::stoull(argv[++i]);
        else if (a == "--kv-capacity" && i + 1 < argc) perf_config_.kv_capacity = std::stoul(argv[++i]);
    }
}

void ConfigManager::set_defaults() {
    memory_config_ = MemoryConfig{};
    perf_config_ = PerformanceConfig{};
    logging_config_ = LoggingConfig{};
    power_config_ = PowerConfig{};
    benchmark_config_ = BenchmarkConfig{};
    codec_config_ = CodecConfig{};
    batch_config_ = BatchConfig{};
    vitality_config_ = VitalityConfig{};
    shader_config_ = ShaderConfig{};
    model_path_.clear();
    model_type_.clear();
    toml_data_.clear();
}

int ConfigManager::get_int(const std::string& s, const std::string& k, int d) const {
    auto it = toml_data_.find(s);
    if (it == toml_data_.end()) return d;
    auto kv = it->second.find(k);
    if (kv == it->second.end() || !std::holds_alternative<int64_t>(kv->second)) return d;
    return static_cast<int>(std::get<int64_t>(kv->second));
}
float ConfigManager::get_float(const std::string& s, const std::string& k, float d) const {
    auto it = toml_data_.find(s);
    if (it == toml_data_.end()) return d;
    auto kv = it->second.find(k);
    if (kv == it->second.end() || !std::holds_alternative<double>(kv->second)) return d;
    return static_cast<float>(std::get<double>(kv->second));
}
bool ConfigManager::get_bool(const std::string& s, const std::string& k, bool d) const {
    auto it = toml_data_.find(s);
    if (it == toml_data_.end()) return d;
    auto kv = it->second.find(k);
    if (kv == it->second.end() || !std::holds_alternative<bool>(kv->second)) return d;
    return std::get<bool>(kv->second);
}
std::string ConfigManager::get_string(const std::string& s, const std::string& k, const std::string& d) const {
    auto it = toml_data_.find(s);
    if (it == toml_data_.end()) return d;
    auto kv = it->second.find(k);
    if (kv == it->second.end() || !std::holds_alternative<std::string>(kv->second)) return d;
    return std::get<std::string>(kv->second);
}

bool ConfigManager::validate_config() const {
    bool ok = true;
    if (memory_config_.vram_budget_gb <= 0.0f || memory_config_.vram_budget_gb > 288.0f) {
        std::cerr << "Error: VRAM budget must be in (0, 288] GB" << std::endl;
        ok = false;
    }
    if (memory_config_.ram_budget_gb <= 0.0f || memory_config_.ram_budget_gb > 4096.0f) {
        std::cerr << "Error: RAM budget must be in (0, 4096] GB" << std::endl;
        ok = false;
    }
    return ok;
}

void ConfigManager::print_config() const {
    std::cout << "=== Vulkan Symbiote Configuration (MI355X backend) ===\n"
              << "Memory: VRAM budget " << memory_config_.vram_budget_gb << " GB, RAM budget "
              << memory_config_.ram_budget_gb << " GB\n"
              << "Performance: GPU " << (perf_config_.enable_gpu ? "enabled" : "disabled") << ", device "
              << perf_config_.device << ", kv_capacity " << perf_config_.kv_capacity << "\n"
              << "Power profile: " << power_config_.power_profile << std::endl;
}

std::string ConfigManager::get_current_timestamp() const {
    auto now = std::chrono::system_clock::to_time_t(std::chrono::system_clock::now());
    std::tm tm{};
    localtime_r(&now, &tm);
    std::ostringstream o;
    o << std::put_time(&tm, "%Y-%m-%dT%H:%M:%S");
    return o.str();
}

}  // namespace vk_symbiote
