#include "engine.hpp"
#include "roctx_range.hpp"

#include <dlfcn.h>
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <cstdlib>
#include <chrono>
#include <cstring>
#include <filesystem>
#include <optional>
#include <fstream>
#include <set>
#include <unordered_set>

namespace fs = std::filesystem;

namespace edge_fm {

// =================================================================================
// Safetensors + WeightLoader
// =================================================================================
std::map<std::string, SafetensorsEntry> read_safetensors_header(const std::string& path, size_t* data_offset) {
    std::ifstream f(path, std::ios::binary);
    if (!f) throw ModelNotLoadedError("cannot open safetensors file: " + path);
    uint64_t n = 0;
    f.read(reinterpret_cast<char*>(&n), 8);
    if (!f || n == 0 || n > (1ull << 31)) throw ModelNotLoadedError("bad safetensors header size: " + path);
    std::string hdr(n, '\0');
    f.read(&hdr[0], (std::streamsize)n);
    if (!f) throw ModelNotLoadedError("truncated safetensors header: " + path);
    std::map<std::string, SafetensorsEntry> out;
    try {
        Json j = Json::parse(hdr);
        for (const auto& kv : j.as_object()) {
            if (kv.first == "__metadata__") continue;
            SafetensorsEntry e;
            e.dtype = kv.second.at("dtype").as_string();
            for (const auto& s : kv.second.at("shape").as_array()) e.shape.push_back(s.as_int());
            const auto& off = kv.second.at("data_offsets").as_array();
            if (off.size() != 2 || off[0].as_int() < 0 || off[1].as_int() < off[0].as_int())
                throw ModelNotLoadedError("bad data_offsets");
            e.begin = (size_t)off[0].as_int();
            e.end = (size_t)off[1].as_int();
            out[kv.first] = e;
        }
    } catch (const std::exception& ex) {
        throw ModelNotLoadedError("malformed safetensors header in " + path + ": " + ex.what());
    }
    *data_offset = 8 + n;
    return out;
}

static DType st_dtype(const std::string& s) {
    if (s == "BF16") return DType::BFloat16;
    if (s == "F16") return DType::Float16;
    if (s == "F32") return DType::Float32;
    if (s == "I32") return DType::Int32;
    if (s == "I64") return DType::Int64;
    if (s == "I8") return DType::Int8;
    if (s == "U8") return DType::UInt8;
    throw ModelNotLoadedError("unsupported safetensors dtype " + s);
}

WeightLoader& WeightLoader::instance() {
    static WeightLoader w;
    return w;
}

std::vector<std::string> collect_safetensors_files(const std::string& model_path) {
    std::vector<std::string> files;
    if (fs::is_regular_file(model_path)) return {model_path};
    const fs::path single = fs::path(model_path) / "model.safetensors";
    if (fs::is_regular_file(single)) return {single.string()};
    if (fs::is_directory(model_path)) {
        for (const auto& e : fs::directory_iterator(model_path)) {
            if (!e.is_regular_file()) continue;
            const std::string name = e.path().filename().string();
            if (name.rfind("model-", 0) == 0 && name.find("-of-") != std::string::npos &&
                e.path().extension() == ".safetensors")
                files.push_back(e.path().string());
        }
    }
    std::sort(files.begin(), files.end());
    if (files.empty())
        throw ConfigurationError("No model.safetensors or model-*-of-*.safetensors found in: " + model_path);
    return files;
}

std::string vl_language_model_name(const std::string& name) {
    auto starts = [&](const char* p) { return name.rfind(p, 0) == 0; };
    if (starts("model.visual.")) return "";   // the vision tower of the newer HF layout
    if (starts("model.language_model.")) return "model." + name.substr(std::strlen("model.language_model."));
    if (starts("model.model.")) return name.substr(std::strlen("model."));
    if (starts("language_model.")) return name.substr(std::strlen("language_model."));
    if (starts("model.") || starts("lm_head.")) return name;
    return "";
}

void WeightLoader::load_weights_from_file(const std::string& model_path, ModelStage stage, int32_t device_id,
                                          bool language_model_only) {
    const std::vector<std::string> files = collect_safetensors_files(model_path);
    hip_check(hipSetDevice(device_id), "hipSetDevice");
    std::unordered_map<std::string, Tensor> loaded;
    for (const auto& path : files) {
        size_t data_off = 0;
        auto entries = read_safetensors_header(path, &data_off);
        int fd = ::open(path.c_str(), O_RDONLY);
        if (fd < 0) throw ModelNotLoadedError("cannot open " + path);
        struct stat st;
        fstat(fd, &st);
        void* map = ::mmap(nullptr, (size_t)st.st_size, PROT_READ, MAP_PRIVATE, fd, 0);
        ::close(fd);
        if (map == MAP_FAILED) throw ModelNotLoadedError("mmap failed for " + path);
        for (const auto& kv : entries) {
            const auto& e = kv.second;
            const std::string name = language_model_only ? vl_language_model_name(kv.first) : kv.first;
            if (name.empty()) continue;
            if (e.begin > e.end || data_off + e.end > (size_t)st.st_size) {
                ::munmap(map, (size_t)st.st_size);
                throw ModelNotLoadedError("tensor " + kv.first + " out of file bounds in " + path);
            }
            Tensor t = Tensor::empty(e.shape, st_dtype(e.dtype), Device::GPU, device_id);
            if (t.nbytes() != e.end - e.begin) {
                ::munmap(map, (size_t)st.st_size);
                throw ModelNotLoadedError("size mismatch for tensor " + kv.first + " in " + path);
            }
            hip_check(hipMemcpy(t.data_ptr(), static_cast<const char*>(map) + data_off + e.begin, t.nbytes(),
                                hipMemcpyHostToDevice),
                      "upload " + kv.first);
            loaded[name] = t;
        }
        ::munmap(map, (size_t)st.st_size);
    }
    std::lock_guard<std::mutex> lock(mu_);
    auto& dst = stages_[(int)stage];
    for (auto& kv : loaded) dst[kv.first] = kv.second;
}

void WeightLoader::register_tensor(ModelStage stage, const std::string& name, const Tensor& t) {
    std::lock_guard<std::mutex> lock(mu_);
    stages_[(int)stage][name] = t;
}

const std::unordered_map<std::string, Tensor>& WeightLoader::get(ModelStage stage) {
    std::lock_guard<std::mutex> lock(mu_);
    return stages_[(int)stage];
}

bool WeightLoader::has_stage(ModelStage stage) {
    std::lock_guard<std::mutex> lock(mu_);
    auto it = stages_.find((int)stage);
    return it != stages_.end() && !it->second.empty();
}

void WeightLoader::clear_stage(ModelStage stage) {
    std::lock_guard<std::mutex> lock(mu_);
    stages_.erase((int)stage);
}

// =================================================================================
// EngineConfig / ModelConfig
// =================================================================================
std::string EngineConfig::default_config_dir() {
    if (const char* env = std::getenv("EDGE_FM_CONFIG_DIR")) return env;
    Dl_info info;
    if (dladdr(reinterpret_cast<void*>(&EngineConfig::default_config_dir), &info) && info.dli_fname) {
        return (fs::path(info.dli_fname).parent_path() / "configs").string();
    }
    return "configs";
}

EngineConfig::EngineConfig(const std::string& config_path) {
    const fs::path def = fs::path(default_config_dir()) / "engine_default.json";
    if (fs::exists(def)) json_ = Json::parse_file(def.string());
    else json_ = Json::object();
    Json user;
    try {
        user = Json::parse_file(config_path);
    } catch (const std::exception& e) {
        throw ConfigurationError(std::string("cannot load engine config: ") + e.what());
    }
    json_.update(user);
    base_dir_ = fs::path(config_path).parent_path().string();
    const std::string mp = prefill_model_path();
    if (mp.empty()) throw ConfigurationError("prefill_model_path is required");
    const fs::path cfgp = fs::path(mp) / "config.json";
    if (!fs::exists(cfgp)) throw ConfigurationError("model config.json not found: " + cfgp.string());
    model_json_ = Json::parse_file(cfgp.string());
}

std::string EngineConfig::model_name() const {
    std::string n = json_.get_string("model_name");
    if (n.empty()) n = model_json_.get_string("model_type", "qwen2_5");
    return normalize_model_name(n);
}
int32_t EngineConfig::device_id() const { return json_.contains("runtime") ? (int32_t)json_.at("runtime").get_int("device_id", 0) : 0; }
std::string EngineConfig::hw_profile() const {
    std::string hw = json_.contains("runtime") ? json_.at("runtime").get_string("hw_profile") : "";
    if (hw.empty() || hw == "auto") hw = "rocm_gfx950";
    return normalize_identifier(hw);
}
bool EngineConfig::use_graph() const {
    if (!json_.contains("runtime")) return true;
    const Json& r = json_.at("runtime");
    if (r.contains("use_hip_graph")) return r.get_bool("use_hip_graph", true);
    return r.get_bool("use_cuda_graph", true);
}
bool EngineConfig::lm_head_top1() const {
    return json_.contains("runtime") ? json_.at("runtime").get_bool("lm_head_top1", true) : true;
}
bool EngineConfig::debug_logits() const {
    return json_.contains("runtime") ? json_.at("runtime").get_bool("debug_logits", false) : false;
}
bool EngineConfig::decode_fused_qkv_attention() const {
    const char* env = std::getenv("EDGE_FM_DECODE_FUSED_QKV_ATTENTION");
    if (env != nullptr && env[0] != '\0') return std::string(env) != "0";
    return json_.contains("runtime") ? json_.at("runtime").get_bool("decode_fused_qkv_attention", true) : true;
}
std::string EngineConfig::operator_table_path() const {
    std::string p = json_.get_string("operator_impl_table_path");
    if (!p.empty() && fs::path(p).is_relative() && !base_dir_.empty()) p = (fs::path(base_dir_) / p).string();
    return p;
}
std::string EngineConfig::prefill_model_path() const {
    std::string p = json_.get_string("prefill_model_path");
    if (!p.empty() && fs::path(p).is_relative() && !base_dir_.empty()) p = (fs::path(base_dir_) / p).string();
    return p;
}
std::vector<KVSlotConfig> EngineConfig::kv_slots() const {
    std::vector<KVSlotConfig> out;
    if (json_.contains("kvcache") && json_.at("kvcache").contains("requests")) {
        for (const auto& r : json_.at("kvcache").at("requests").as_array()) {
            KVSlotConfig s;
            s.request_id = (int32_t)r.get_int("request_id", 0);
            s.max_tokens = (int32_t)r.get_int("max_tokens", 4096);
            if (r.contains("prefix_token_ids"))
                for (const auto& t : r.at("prefix_token_ids").as_array()) s.prefix_token_ids.push_back((int32_t)t.as_int());
            out.push_back(s);
        }
    }
    if (out.empty()) out.push_back(KVSlotConfig{});
    return out;
}
int32_t EngineConfig::max_new_tokens() const {
    return json_.contains("sampling") ? (int32_t)json_.at("sampling").get_int("max_new_tokens", 256) : 256;
}
float EngineConfig::temperature() const {
    return json_.contains("sampling") ? (float)json_.at("sampling").get_double("temperature", 1.0) : 1.0f;
}
float EngineConfig::top_p() const {
    return json_.contains("sampling") ? (float)json_.at("sampling").get_double("top_p", 1.0) : 1.0f;
}
uint64_t EngineConfig::seed() const {
    return json_.contains("sampling") ? (uint64_t)json_.at("sampling").get_int("seed", 0) : 0;
}
std::vector<int32_t> EngineConfig::stop_token_ids() const {
    std::vector<int32_t> out;
    if (json_.contains("sampling") && json_.at("sampling").contains("stop_token_ids"))
        for (const auto& t : json_.at("sampling").at("stop_token_ids").as_array()) out.push_back((int32_t)t.as_int());
    return out;
}
std::vector<int32_t> EngineConfig::eos_token_ids() const {
    std::vector<int32_t> out;
    auto add = [&](const Json& j) {
        if (!j.contains("eos_token_id")) return;
        const Json& e = j.at("eos_token_id");
        if (e.is_number()) out.push_back((int32_t)e.as_int());
        else if (e.is_array())
            for (const auto& t : e.as_array()) out.push_back((int32_t)t.as_int());
    };
    add(model_json_);
    const fs::path gen = fs::path(prefill_model_path()) / "generation_config.json";
    if (fs::exists(gen)) add(Json::parse_file(gen.string()));
    return out;
}

Json EngineConfig::compact_vocab() const {
    if (json_.contains("compact_vocab") && json_.at("compact_vocab").is_object()) return json_.at("compact_vocab");
    return Json::object();
}

ModelConfig ModelConfig::from_json(const Json& j0) {
    // Qwen2.5-VL keeps the language model hyper-parameters under text_config.
    const Json& j = j0.contains("text_config") ? j0.at("text_config") : j0;
    ModelConfig m;
    m.hidden = (int32_t)j.get_int("hidden_size", 0);
    m.inter = (int32_t)j.get_int("intermediate_size", 0);
    m.layers = (int32_t)j.get_int("num_hidden_layers", 0);
    m.heads = (int32_t)j.get_int("num_attention_heads", 0);
    m.kv_heads = (int32_t)j.get_int("num_key_value_heads", m.heads);
    m.head_dim = (int32_t)j.get_int("head_dim", m.heads ? m.hidden / m.heads : 0);
    m.vocab = j.get_int("vocab_size", j0.get_int("vocab_size", 0));
    m.eps = (float)j.get_double("rms_norm_eps", 1e-6);
    double theta = j.get_double("rope_theta", 0.0);
    if (theta == 0.0 && j.contains("rope_parameters")) theta = j.at("rope_parameters").get_double("rope_theta", 0.0);
    m.theta = (float)(theta > 0.0 ? theta : 1.0e6);
    m.tied = j0.get_bool("tie_word_embeddings", j.get_bool("tie_word_embeddings", true));
    const Json* rs = nullptr;
    if (j.contains("rope_scaling") && j.at("rope_scaling").is_object()) rs = &j.at("rope_scaling");
    else if (j0.contains("rope_scaling") && j0.at("rope_scaling").is_object()) rs = &j0.at("rope_scaling");
    if (rs && rs->contains("mrope_section")) {
        const auto& s = rs->at("mrope_section").as_array();
        check<ConfigurationError>(s.size() == 3, "mrope_section must have 3 entries");
        for (int i = 0; i < 3; ++i) m.mrope_section[i] = (int32_t)s[i].as_int();
        m.mrope = true;
    }
    check<ConfigurationError>(m.hidden > 0 && m.layers > 0 && m.heads > 0 && m.kv_heads > 0 && m.vocab > 0 &&
                                  m.inter > 0,
                              "incomplete model config.json");
    const std::string td = j0.get_string("torch_dtype", j.get_string("torch_dtype", "bfloat16"));
    check<ConfigurationError>(td == "bfloat16" || td == "bf16",
                              "the gfx950 kernels run bf16 models (torch_dtype " + td + ")");
    return m;
}

// =================================================================================
// KVManager
// =================================================================================
KVManager::KVManager(const std::vector<KVSlotConfig>& slots, const ModelConfig& m, int32_t device_id)
    : m_(m), device_id_(device_id) {
    std::set<int32_t> seen;
    for (const auto& s : slots) {
        check<ConfigurationError>(seen.insert(s.request_id).second, "duplicate kvcache request_id");
        check<ConfigurationError>(s.max_tokens > 0, "kvcache max_tokens must be positive");
        check<ConfigurationError>((int32_t)s.prefix_token_ids.size() < s.max_tokens, "prefix longer than max_tokens");
        KVSlot slot;
        slot.cfg = s;
        slot.prefix_size = (int32_t)s.prefix_token_ids.size();
        slot.buffer = Tensor::zeros({(int64_t)m.layers, 2, (int64_t)s.max_tokens, (int64_t)m.kv_dim()},
                                    DType::BFloat16, Device::GPU, device_id);
        slots_.push_back(std::move(slot));
    }
}

KVSlot& KVManager::slot(int32_t request_id) {
    for (auto& s : slots_)
        if (s.cfg.request_id == request_id) return s;
    throw InvalidRequestError("Invalid request_id: " + std::to_string(request_id));
}
bool KVManager::is_request_valid(int32_t request_id) const {
    for (const auto& s : slots_)
        if (s.cfg.request_id == request_id) return true;
    return false;
}
void* KVManager::k_cache(int32_t request_id, int layer) {
    KVSlot& s = slot(request_id);
    const size_t per = (size_t)s.cfg.max_tokens * m_.kv_dim() * 2;
    return static_cast<char*>(s.buffer.data_ptr()) + (size_t)layer * 2 * per;
}
void* KVManager::v_cache(int32_t request_id, int layer) {
    KVSlot& s = slot(request_id);
    const size_t per = (size_t)s.cfg.max_tokens * m_.kv_dim() * 2;
    return static_cast<char*>(s.buffer.data_ptr()) + ((size_t)layer * 2 + 1) * per;
}
std::vector<int32_t> KVManager::request_ids() const {
    std::vector<int32_t> out;
    for (const auto& s : slots_) out.push_back(s.cfg.request_id);
    return out;
}

namespace {
std::vector<KVSlotConfig> remapped_slots(const EngineConfig& cfg) {
    const CompactVocab vocab(cfg);
    std::vector<KVSlotConfig> slots = cfg.kv_slots();
    check<ConfigurationError>(!slots.empty(), "kvcache.requests array must not be empty");
    for (auto& s : slots)
        s.prefix_token_ids = vocab.remap_required_token_ids(s.prefix_token_ids, "kvcache.requests[].prefix_token_ids");
    return slots;
}
}  // namespace

KVManager::KVManager(const EngineConfig& cfg)
    : KVManager(remapped_slots(cfg), ModelConfig::from_json(cfg.model_config()), cfg.device_id()) {}

const KVSlot& KVManager::find(int32_t request_id) const {
    for (const auto& s : slots_)
        if (s.cfg.request_id == request_id) return s;
    throw InvalidRequestError("Invalid request_id: " + std::to_string(request_id));
}

std::vector<void*> KVManager::get_read_kvcache(int32_t request_id) const {
    const KVSlot& s = find(request_id);
    const size_t layer_bytes = 2 * (size_t)s.cfg.max_tokens * (size_t)m_.kv_dim() * 2;
    std::vector<void*> out((size_t)m_.layers);
    for (int l = 0; l < m_.layers; ++l) out[l] = static_cast<char*>(s.buffer.data_ptr()) + (size_t)l * layer_bytes;
    return out;
}

std::vector<void*> KVManager::get_write_kvcache(int32_t request_id) const {
    const KVSlot& s = find(request_id);
    std::vector<void*> out = get_read_kvcache(request_id);
    const size_t prefix_bytes = (size_t)s.prefix_size * (size_t)m_.kv_dim() * 2;
    for (auto& p : out) p = static_cast<char*>(p) + prefix_bytes;
    return out;
}

KVManagerStatus KVManager::get_status() const {
    KVManagerStatus st;
    st.device = Device::GPU;
    st.device_id = device_id_;
    for (const auto& s : slots_) {
        KVSlotStatus k;
        k.request_id = s.cfg.request_id;
        k.prefix_token_ids = s.cfg.prefix_token_ids;
        k.prefix_size = (size_t)s.prefix_size;
        k.max_tokens = s.cfg.max_tokens;
        k.allocated_size = s.buffer.nbytes();
        st.slots.push_back(std::move(k));
    }
    return st;
}

// =================================================================================
// Qwen2_5
// =================================================================================
const Tensor& Qwen2_5::w(const std::unordered_map<std::string, Tensor>& ws, const std::string& name) const {
    // Registered tensors may keep a Qwen2.5-VL checkpoint's names (engine_factory.cpp:73-98):
    // model.X is also looked up as model.language_model.X, model.model.X and
    // language_model.model.X, lm_head.X as language_model.lm_head.X.
    auto it = ws.find(name);
    if (it != ws.end()) return it->second;
    const bool under_model = name.rfind("model.", 0) == 0;
    const std::string rest = under_model ? name.substr(6) : name;
    const std::vector<std::string> alts =
        under_model ? std::vector<std::string>{"model.language_model." + rest, "model.model." + rest,
                                               "language_model.model." + rest}
                    : std::vector<std::string>{"language_model." + name};
    for (const auto& key : alts) {
        it = ws.find(key);
        if (it != ws.end()) return it->second;
    }
    throw ModelNotLoadedError("missing weight tensor: " + name);
}

Tensor concat_rows(const std::vector<const Tensor*>& parts, int32_t device_id, hipStream_t s) {
    int64_t rows = 0, cols = -1;
    for (auto* p : parts) {
        check<ModelNotLoadedError>(p->dtype() == DType::BFloat16, "weights must be bf16");
        const int64_t c = p->shape().size() == 2 ? p->shape()[1] : 1;
        check<ModelNotLoadedError>(cols < 0 || c == cols, "fused weight column mismatch");
        cols = c;
        rows += p->shape()[0];
    }
    Tensor out = parts[0]->shape().size() == 2 ? Tensor::empty({rows, cols}, DType::BFloat16, Device::GPU, device_id)
                                               : Tensor::empty({rows}, DType::BFloat16, Device::GPU, device_id);
    size_t off = 0;
    for (auto* p : parts) {
        hip_check(hipMemcpyAsync(static_cast<char*>(out.data_ptr()) + off, p->data_ptr(), p->nbytes(),
                                 hipMemcpyDeviceToDevice, s),
                  "fuse weights");
        off += p->nbytes();
    }
    return out;
}

Qwen2_5::Qwen2_5(const EngineConfig& cfg, const ModelConfig& m, const std::unordered_map<std::string, Tensor>& ws,
                 int32_t device_id)
    : cfg_(cfg), m_(m), device_id_(device_id) {
    model_name_ = cfg.model_name();
    hw_profile_ = cfg.hw_profile();
    fused_front_enabled_ = cfg.decode_fused_qkv_attention() && !m.mrope;
    table_path_ = cfg.operator_table_path();
    hip_check(hipSetDevice(device_id), "hipSetDevice");
    check<ConfigurationError>(m.hidden % 8 == 0 && m.inter % 8 == 0 && m.q_dim() % 8 == 0,
                              "hidden / intermediate sizes must be multiples of 8");

    // ---- operator resolution (attention.cu:211-276, linear_impl.cu:866-915) ----
    auto resolve = [&](const char* kind, const char* stage) {
        OperatorQuery q;
        q.op_kind = kind;
        q.stage = stage;
        return resolve_impl_id(model_name_, hw_profile_, table_path_, q);
    };
    AttentionOpContext actx = attn_ctx();
    attn_ = AttentionOpRegistry::instance().find_impl_by_id(resolve("attention", "prefill"));
    if (attn_ == nullptr || !attn_->supports(actx)) attn_ = AttentionOpRegistry::instance().default_impl(actx);
    RMSNormOpContext nctx;
    nctx.hidden_size = (uint32_t)m.hidden;
    norm_ = NormOpRegistry::instance().find_impl_by_id(resolve("norm", "prefill"));
    if (norm_ == nullptr || !norm_->supports(nctx)) norm_ = NormOpRegistry::instance().default_impl(nctx);
    ActivationOpContext act;
    act.hidden_size = m.inter;
    act.input_layout = ActivationInputLayout::kUpGate;
    act_ = ActivationOpRegistry::instance().find_impl_by_id(resolve("activation", "prefill"));
    if (act_ == nullptr || !act_->supports(act)) act_ = ActivationOpRegistry::instance().default_impl(act);
    FusedGateUpActivationContext gctx;
    gctx.stage = ModelStage::Prefill;
    gctx.m = 2;
    gctx.hidden = m.hidden;
    gctx.intermediate = m.inter;
    swiglu_ = FusedGateUpActivationRegistry::instance().find_impl_by_id(resolve("fused_gate_up_activation", "prefill"));
    if (swiglu_ == nullptr) swiglu_ = FusedGateUpActivationRegistry::instance().default_impl(gctx);

    // ---- weights: fused layouts (linear.cu:1629-1785, 1923-1943, 2239-2286) ----
    hipStream_t s = nullptr;
    embed_ = w(ws, "model.embed_tokens.weight");
    check<ModelNotLoadedError>(embed_.shape().size() == 2 && embed_.shape()[0] == m.vocab &&
                                   embed_.shape()[1] == m.hidden,
                               "embed_tokens shape mismatch");
    final_norm_ = w(ws, "model.norm.weight");
    auto lm = ws.find("lm_head.weight");
    lm_head_ = (!m.tied && lm != ws.end()) ? lm->second : embed_;
    if (lm != ws.end() && !m.tied) lm_head_ = lm->second;
    for (int l = 0; l < m.layers; ++l) {
        const std::string p = "model.layers." + std::to_string(l) + ".";
        Layer L;
        L.qkv_w = concat_rows({&w(ws, p + "self_attn.q_proj.weight"), &w(ws, p + "self_attn.k_proj.weight"),
                               &w(ws, p + "self_attn.v_proj.weight")},
                              device_id, s);
        check<ModelNotLoadedError>(L.qkv_w.shape()[0] == m.q_dim() + 2 * m.kv_dim() && L.qkv_w.shape()[1] == m.hidden,
                                   "qkv weight shape mismatch");
        L.qkv_b = concat_rows({&w(ws, p + "self_attn.q_proj.bias"), &w(ws, p + "self_attn.k_proj.bias"),
                               &w(ws, p + "self_attn.v_proj.bias")},
                              device_id, s);
        L.o_w = w(ws, p + "self_attn.o_proj.weight");
        L.gu_w = concat_rows({&w(ws, p + "mlp.up_proj.weight"), &w(ws, p + "mlp.gate_proj.weight")}, device_id, s);
        L.down_w = w(ws, p + "mlp.down_proj.weight");
        L.in_norm = w(ws, p + "input_layernorm.weight");
        L.post_norm = w(ws, p + "post_attention_layernorm.weight");
        const uint32_t H = (uint32_t)m.hidden, QD = (uint32_t)m.q_dim(), KVD = (uint32_t)m.kv_dim(),
                       I = (uint32_t)m.inter;
        const std::string n = "Layer_" + std::to_string(l);
        L.qkv = std::make_unique<FusedQKVLinearLayer>(p + "self_attn", cfg, H, QD, KVD, KVD, n + "_QKVLinear");
        L.o_proj = std::make_unique<LinearLayer>(p + "self_attn.o_proj", cfg, QD, H, n + "_OProj");
        L.gate_up = std::make_unique<FusedGateUpLinearLayer>(p + "mlp", cfg, H, I, I, n + "_GateUp");
        L.down = std::make_unique<LinearLayer>(p + "mlp.down_proj", cfg, I, H, n + "_DownProj");
        L.qkv->load_weights(L.qkv_w, &L.qkv_b);
        L.o_proj->load_weights(L.o_w, nullptr);
        L.gate_up->load_weights(L.gu_w, nullptr);
        L.down->load_weights(L.down_w, nullptr);
        layers_.push_back(std::move(L));
    }
    mlp_source_ = std::make_unique<PrefillMlpSourceOp>(cfg);
    hip_check(hipDeviceSynchronize(), "fuse weights");

    // ---- decode scratch ----
    const int64_t H = m.hidden;
    dec_h_ = Tensor::zeros({1, H}, DType::BFloat16, Device::GPU, device_id);
    dec_res_[0] = Tensor::zeros({1, H}, DType::BFloat16, Device::GPU, device_id);
    dec_res_[1] = Tensor::zeros({1, H}, DType::BFloat16, Device::GPU, device_id);
    dec_q_ = Tensor::zeros({1, (int64_t)m.q_dim()}, DType::BFloat16, Device::GPU, device_id);
    dec_attn_ = Tensor::zeros({1, (int64_t)m.q_dim()}, DType::BFloat16, Device::GPU, device_id);
    dec_a_ = Tensor::zeros({1, H}, DType::BFloat16, Device::GPU, device_id);
    dec_mid_ = Tensor::zeros({1, (int64_t)m.inter}, DType::BFloat16, Device::GPU, device_id);
    dec_kvtmp_ = Tensor::zeros({2, (int64_t)m.kv_dim()}, DType::BFloat16, Device::GPU, device_id);
    dec_one_ = Tensor::empty({1}, DType::Int32, Device::GPU, device_id);
    const uint32_t one = 1;
    hip_check(hipMemcpy(dec_one_.data_ptr(), &one, 4, hipMemcpyHostToDevice), "init");
    top1_ws_ = Tensor::zeros({(int64_t)efm_lm_head_top1_workspace_bytes(m.vocab)}, DType::UInt8, Device::GPU, device_id);
}

void Qwen2_5::reserve_decode(uint32_t max_kv_len) {
    const efm_attention_ctx c = decode_ctx();
    const size_t bytes = efm_attention_decode_workspace_bytes(&c, max_kv_len);
    if (attn_ws_.empty() || attn_ws_.nbytes() < bytes)
        attn_ws_ = Tensor::zeros({(int64_t)bytes}, DType::UInt8, Device::GPU, device_id_);
    // the decode plan for this cache length (impls resolved, their scratch prepared):
    // nothing is resolved or allocated while a decode step is captured
    if (!plans_.count(max_kv_len)) {
        std::vector<DecodeLayerPlan> plan;
        for (int l = 0; l < m_.layers; ++l) {
            Layer& Ly = layers_[l];
            plan.push_back(resolve_decode_layer(cfg_, m_, l, max_kv_len, fused_front_enabled_, *Ly.o_proj, *Ly.down));
            if (plan.back().gate_up.empty()) Ly.gate_up->selected_impl_id(ModelStage::Decode, 1);
        }
        plans_.emplace(max_kv_len, std::move(plan));
    }
    const auto& plan = plans_.at(max_kv_len);
    if (uses_fused_front(max_kv_len) && front_sync_ws_.empty()) {
        const size_t sb = efm_decode_qkv_attention_sync_bytes(m_.q_dim(), m_.kv_dim());
        front_sync_ws_ = Tensor::zeros({(int64_t)sb}, DType::UInt8, Device::GPU, device_id_);
    }
    for (const auto& p : plan)
        if (p.gate_up.empty() && dec_gu_.empty())
            dec_gu_ = Tensor::zeros({1, 2 * (int64_t)m_.inter}, DType::BFloat16, Device::GPU, device_id_);
}

const std::vector<DecodeLayerPlan>& Qwen2_5::decode_plan(uint32_t max_kv_len) const {
    auto it = plans_.find(max_kv_len);
    check<InternalError>(it != plans_.end(), "decode plan not resolved for this cache length");
    return it->second;
}

// Some layer runs the fused norm + QKV + attention partials launch (text models whose
// cache needs at most 8 splits; the merge folds into the o_proj prologue).
bool Qwen2_5::uses_fused_front(uint32_t max_kv_len) const {
    auto it = plans_.find(max_kv_len);
    if (it == plans_.end()) return false;
    for (const auto& p : it->second)
        if (p.attention == "hip_gfx950_decode_fused_qkv_attention") return true;
    return false;
}

void Qwen2_5::check_decode_status(hipStream_t stream) {
    if (!front_sync_ws_.empty())
        efm_check(efm_decode_qkv_attention_status(front_sync_ws_.data_ptr(), stream), "decode qkv + attention");
}

AttentionOpContext Qwen2_5::attn_ctx() const {
    AttentionOpContext c;
    c.num_qo_heads = (uint32_t)m_.heads;
    c.num_kv_heads = (uint32_t)m_.kv_heads;
    c.head_dim = (uint32_t)m_.head_dim;
    c.rope_theta = m_.theta;
    c.rope_scale = 1.0f;
    c.dtype = DType::BFloat16;
    // Text models rotate inside attention; M-RoPE models rotate before the cache write
    // (src/layers/attention.cu:135-139).
    c.pos_encoding = m_.mrope ? AttentionPosEncoding::kNone : AttentionPosEncoding::kRoPELlama;
    c.device_id = device_id_;
    return c;
}

efm_attention_ctx Qwen2_5::decode_ctx() const {
    efm_attention_ctx c = to_c_ctx(attn_ctx());
    // text models: the cache holds keys rotated at their positions (prefill rotates
    // them before the cache write); this step's key, written un-rotated by the QKV
    // projection of the fused front half, is rotated by the attention
    // call that first reads it
    if (!m_.mrope) c.k_already_prerotated = EFM_K_PREROTATED_EXCEPT_NEWEST;
    return c;
}

efm_attention_ctx Qwen2_5::decode_attn_ctx_rotated() const {
    // every key in the cache and q already rotated (efm_decode_norm_qkv_rope, or the
    // M-RoPE write): the attention itself applies no positional encoding
    efm_attention_ctx c = to_c_ctx(attn_ctx());
    c.pos_encoding = EFM_POS_NONE;
    c.k_already_prerotated = 0;
    return c;
}

uint64_t Qwen2_5::prefill_buffers_epoch() const {
    return pf_epoch_ + mlp_source_->generation() + linear_scratch_generation(device_id_);
}

void Qwen2_5::ensure_prefill_capacity(int32_t S) {
    if (S <= pf_cap_) return;
    ++pf_epoch_;
    const int64_t n = std::max<int64_t>(S, 64);
    const int64_t H = m_.hidden;
    pf_hidden_ = Tensor::empty({n, H}, DType::BFloat16, Device::GPU, device_id_);
    pf_res_ = Tensor::empty({n, H}, DType::BFloat16, Device::GPU, device_id_);
    pf_norm_ = Tensor::empty({n, H}, DType::BFloat16, Device::GPU, device_id_);
    pf_qkv_ = Tensor::empty({n, (int64_t)(m_.q_dim() + 2 * m_.kv_dim())}, DType::BFloat16, Device::GPU, device_id_);
    pf_attn_ = Tensor::empty({n, (int64_t)m_.q_dim()}, DType::BFloat16, Device::GPU, device_id_);
    pf_mid_ = Tensor::empty({n, (int64_t)m_.inter}, DType::BFloat16, Device::GPU, device_id_);
    pf_cap_ = (int32_t)n;
}

void Qwen2_5::prefill(int32_t S, int32_t base, const int32_t* ids, const Tensor* emb, int32_t embed_token_id,
                      const int32_t* position_ids, void** k_caches, void** v_caches, int32_t* token_out, float* logits,
                      hipStream_t stream) {
    ensure_prefill_capacity(S);
    const int64_t H = m_.hidden, QD = m_.q_dim(), KVD = m_.kv_dim(), TOT = QD + 2 * KVD;
    const int32_t L = base + S;
    // 1. embedding (embed_head.cu:135-164)
    efm_check(efm_embedding_lookup(S, H, m_.vocab, ids, embed_.data_ptr(), emb ? emb->data_ptr() : nullptr,
                                   emb ? emb->shape()[0] : 0, embed_token_id, pf_hidden_.data_ptr(), stream),
              "prefill embedding");
    RMSNormOpContext nctx;
    nctx.batch_size = (uint32_t)S;
    nctx.hidden_size = (uint32_t)H;
    nctx.eps = m_.eps;
    // Q and K are rotated before attention (M-RoPE, or RoPE at positions base + i for
    // text models, qwen2_5.cpp:807-830), so the cache holds rotated keys and the
    // attention kernels apply no rotation.
    AttentionOpContext actx = attn_ctx();
    actx.q_stride_n = (uint32_t)TOT;
    actx.q_stride_h = (uint32_t)m_.head_dim;
    actx.pos_encoding = AttentionPosEncoding::kNone;
    const size_t row = (size_t)KVD * 2;
    for (int l = 0; l < m_.layers; ++l) {
        const Layer& Ly = layers_[l];
        Tensor hid = pf_hidden_.prefix_view({S, H}), nrm = pf_norm_.prefix_view({S, H}), res = pf_res_.prefix_view({S, H});
        // 2a. input norm (qwen2_5.cpp:564-576)
        if (l == 0) {
            norm_->rms_norm_forward_fn()(nctx, hid, Ly.in_norm, nrm, stream);
            hip_check(hipMemcpyAsync(res.data_ptr(), hid.data_ptr(), (size_t)S * H * 2, hipMemcpyDeviceToDevice,
                                     stream),
                      "save residual");
        } else {
            norm_->fused_add_rms_norm_forward_fn()(nctx, nrm, res, Ly.in_norm, stream);
        }
        // 2b. fused QKV projection + bias
        Tensor qkv = pf_qkv_.prefix_view({S, TOT});
        Ly.qkv->forward_fp16_bf16(nrm, qkv, stream, ModelStage::Prefill);
        // 2c. K / V rows into cache rows [base, base + S) (qwen2_5.cpp:743-746)
        char* kc = static_cast<char*>(k_caches[l]);
        char* vc = static_cast<char*>(v_caches[l]);
        // rotate q in the fused buffer, rotate K into the cache rows [base, base + S) and
        // copy V there, in one pass (attention.cu:17-118 for M-RoPE; text models rotate
        // at position base + t)
        efm_check(efm_prefill_rope_write_kv(qkv.data_ptr(), (int32_t)TOT, kc + (size_t)base * row,
                                            vc + (size_t)base * row, (int32_t)KVD, S, m_.heads, m_.kv_heads,
                                            m_.head_dim, m_.mrope ? position_ids : nullptr, S, m_.mrope ? 0 : base,
                                            m_.mrope_section[0], m_.mrope_section[1], m_.mrope_section[2], m_.theta,
                                            1.0f, stream),
                  "prefill rope + kv write");
        // 2d. attention over cache rows [0, L)
        Tensor qv = Tensor::view(qkv.data_ptr(), {S, m_.heads, m_.head_dim}, DType::BFloat16, Device::GPU, device_id_);
        Tensor kv_k = Tensor::view(kc, {L, m_.kv_heads, m_.head_dim}, DType::BFloat16, Device::GPU, device_id_);
        Tensor kv_v = Tensor::view(vc, {L, m_.kv_heads, m_.head_dim}, DType::BFloat16, Device::GPU, device_id_);
        Tensor ao = pf_attn_.prefix_view({S, QD});
        attn_->forward_prefill(actx, qv, kv_k, kv_v, ao, true, stream);
        // 2e. o_proj -> hidden, post-attention fused add + norm
        Ly.o_proj->forward_fp16_bf16(ao, hid, stream, ModelStage::Prefill);
        norm_->fused_add_rms_norm_forward_fn()(nctx, hid, res, Ly.post_norm, stream);
        // 2f. MLP into the next layer's norm input (or hidden for the last layer),
        // qwen2_5.cpp:855-875: the prefill MLP source op (gate/up GEMM with its SwiGLU
        // epilogue, then down), else the layered path (GatedMlpLayer, gated_mlp.cu:19-67)
        Tensor dst = (l < m_.layers - 1) ? nrm : hid;
        if (!mlp_source_->try_forward(l, hid, Ly.gu_w, Ly.down_w, dst, stream)) {
            Tensor mid = pf_mid_.prefix_view({S, (int64_t)m_.inter});
            FusedGateUpActivationContext gctx;
            gctx.stage = ModelStage::Prefill;
            gctx.m = S;
            gctx.hidden = H;
            gctx.intermediate = m_.inter;
            if (swiglu_ == nullptr || !swiglu_->run(gctx, Ly.gu_w, hid, mid, stream)) {
                Tensor gu = Tensor::empty({S, 2 * (int64_t)m_.inter}, DType::BFloat16, Device::GPU, device_id_);
                Ly.gate_up->forward_fp16_bf16(hid, gu, stream, ModelStage::Prefill);
                ActivationOpContext actx2;
                actx2.batch_size = S;
                actx2.hidden_size = m_.inter;
                actx2.input_layout = ActivationInputLayout::kUpGate;
                act_->act_and_mul(actx2, gu, mid, stream);
            }
            Ly.down->forward_fp16_bf16(mid, dst, stream, ModelStage::Prefill);
        }
    }
    // 3-4. final norm + LM head on the last row (qwen2_5.cpp:883-929)
    const size_t last = (size_t)(S - 1) * H * 2;
    const char* h_last = static_cast<const char*>(pf_hidden_.data_ptr()) + last;
    const char* r_last = static_cast<const char*>(pf_res_.data_ptr()) + last;
    if (logits == nullptr) {
        efm_check(efm_decode_norm_lm_head_top1(m_.hidden, m_.vocab, m_.eps, h_last, r_last, final_norm_.data_ptr(),
                                               lm_head_.data_ptr(), token_out, top1_ws_.data_ptr(), top1_ws_.nbytes(),
                                               stream),
                  "prefill lm head top1");
    } else {
        // final fused add + norm on the last row, then fp32 logits
        hip_check(hipMemcpyAsync(dec_h_.data_ptr(), h_last, H * 2, hipMemcpyDeviceToDevice, stream), "copy");
        hip_check(hipMemcpyAsync(dec_res_[1].data_ptr(), r_last, H * 2, hipMemcpyDeviceToDevice, stream), "copy");
        efm_check(efm_fused_add_rms_norm(1, (uint32_t)H, m_.eps, dec_h_.data_ptr(), dec_res_[1].data_ptr(),
                                         final_norm_.data_ptr(), stream),
                  "prefill final norm");
        efm_check(efm_linear(1, H, m_.vocab, dec_h_.data_ptr(), lm_head_.data_ptr(), nullptr, logits, EFM_DTYPE_F32,
                             stream),
                  "prefill lm head");
    }
}

void Qwen2_5::decode_step(int32_t* token_buf, const uint32_t* d_kv_len, uint32_t max_kv_len, const int32_t* d_pos3,
                          void** k_caches, void** v_caches, float* logits, hipStream_t stream) {
    const int32_t H = m_.hidden, QD = m_.q_dim(), KVD = m_.kv_dim();
    // embedding of the previous token (qwen2_5.cpp:541-549)
    efm_check(efm_embedding_lookup(1, H, m_.vocab, token_buf, embed_.data_ptr(), nullptr, 0, -1, dec_h_.data_ptr(),
                                   stream),
              "decode embedding");
    const efm_attention_ctx c = decode_ctx();
    check<InternalError>(!attn_ws_.empty() && attn_ws_.nbytes() >= efm_attention_decode_workspace_bytes(&c, max_kv_len),
                         "decode workspace not reserved for this cache length");
    const std::vector<DecodeLayerPlan>& plan = decode_plan(max_kv_len);
    const efm_attention_ctx cr = decode_attn_ctx_rotated();
    for (int l = 0; l < m_.layers; ++l) {
        Layer& Ly = layers_[l];
        const DecodeLayerPlan& P = plan[l];
        if (P.attention == "hip_gfx950_decode_fused_qkv_attention") {
            // input norm (+ residual) + QKV + attention split partials in one launch
            efm_check(efm_decode_norm_qkv_attention(
                          &c, H, m_.eps, dec_h_.data_ptr(), (l == 0) ? nullptr : dec_res_[1].data_ptr(),
                          dec_res_[0].data_ptr(), Ly.in_norm.data_ptr(), Ly.qkv_w.data_ptr(), Ly.qkv_b.data_ptr(),
                          k_caches[l], v_caches[l], d_kv_len, max_kv_len, attn_ws_.data_ptr(), attn_ws_.nbytes(),
                          front_sync_ws_.data_ptr(), front_sync_ws_.nbytes(), stream),
                      "decode norm+qkv+attention");
        } else {
            // input norm (+ residual) + QKV + bias, K/V straight into the cache slot
            void* kdst = k_caches[l];
            void* vdst = v_caches[l];
            const uint32_t* slot_len = d_kv_len;
            if (m_.mrope) {  // M-RoPE rotates K before the cache write: stage through kvtmp
                kdst = dec_kvtmp_.data_ptr();
                vdst = static_cast<char*>(dec_kvtmp_.data_ptr()) + (size_t)KVD * 2;
                slot_len = static_cast<const uint32_t*>(dec_one_.data_ptr());
            }
            if (m_.mrope) {
                efm_check(efm_decode_norm_qkv(H, QD, KVD, m_.eps, dec_h_.data_ptr(),
                                              (l == 0) ? nullptr : dec_res_[1].data_ptr(), dec_res_[0].data_ptr(),
                                              Ly.in_norm.data_ptr(), Ly.qkv_w.data_ptr(), Ly.qkv_b.data_ptr(),
                                              dec_q_.data_ptr(), kdst, vdst, slot_len, stream),
                          "decode norm+qkv");
            } else {
                // q and this step's key rotated in the projection's epilogue (the key
                // straight into the cache slot)
                const efm_attention_ctx cq = to_c_ctx(attn_ctx());
                efm_check(efm_decode_norm_qkv_rope(&cq, H, m_.eps, dec_h_.data_ptr(),
                                                   (l == 0) ? nullptr : dec_res_[1].data_ptr(), dec_res_[0].data_ptr(),
                                                   Ly.in_norm.data_ptr(), Ly.qkv_w.data_ptr(), Ly.qkv_b.data_ptr(),
                                                   dec_q_.data_ptr(), kdst, vdst, slot_len, stream),
                          "decode norm+qkv+rope");
            }
            if (m_.mrope) {
                efm_check(efm_decode_mrope_write_kv(dec_q_.data_ptr(), kdst, vdst, dec_q_.data_ptr(), k_caches[l],
                                                    v_caches[l], m_.heads, m_.kv_heads, m_.head_dim, d_pos3,
                                                    m_.mrope_section[0], m_.mrope_section[1], m_.mrope_section[2],
                                                    m_.theta, 1.0f, d_kv_len, stream),
                          "decode mrope + kv write");
            }
            if (P.partials_to_o_proj) {
                efm_check(efm_decode_attention_partials(&cr, dec_q_.data_ptr(), k_caches[l], v_caches[l], d_kv_len,
                                                        max_kv_len, attn_ws_.data_ptr(), attn_ws_.nbytes(), stream),
                          "decode attention partials");
            } else {
                efm_check(efm_attention_decode(&cr, dec_q_.data_ptr(), k_caches[l], v_caches[l], dec_attn_.data_ptr(),
                                               0, d_kv_len, max_kv_len, attn_ws_.data_ptr(), attn_ws_.nbytes(),
                                               stream),
                          "decode attention");
            }
        }
        if (P.partials_to_o_proj) {
            efm_check(efm_decode_attention_merge_o_proj(&c, d_kv_len, max_kv_len, attn_ws_.data_ptr(),
                                                        attn_ws_.nbytes(), Ly.o_w.data_ptr(), H, dec_a_.data_ptr(),
                                                        stream),
                      "decode attention merge + o_proj");
        } else {
            Ly.o_proj->forward_fp16_bf16(dec_attn_, dec_a_, stream, ModelStage::Decode);
        }
        if (!P.gate_up.empty()) {
            efm_check(efm_decode_norm_gate_up_swiglu(H, m_.inter, m_.eps, dec_a_.data_ptr(), dec_res_[0].data_ptr(),
                                                     dec_res_[1].data_ptr(), Ly.post_norm.data_ptr(),
                                                     Ly.gu_w.data_ptr(), dec_mid_.data_ptr(), stream),
                      "decode norm+gate_up+swiglu");
        } else {
            // layered: residual_out <- a + residual_in, a <- norm(.), gate/up, activation
            hip_check(hipMemcpyAsync(dec_res_[1].data_ptr(), dec_res_[0].data_ptr(), (size_t)H * 2,
                                     hipMemcpyDeviceToDevice, stream),
                      "decode residual");
            efm_check(efm_fused_add_rms_norm(1, (uint32_t)H, m_.eps, dec_a_.data_ptr(), dec_res_[1].data_ptr(),
                                             Ly.post_norm.data_ptr(), stream),
                      "decode post-attention norm");
            Ly.gate_up->forward_fp16_bf16(dec_a_, dec_gu_, stream, ModelStage::Decode);
            efm_check(efm_act_and_mul(1, m_.inter, EFM_LAYOUT_UP_GATE, dec_gu_.data_ptr(), dec_mid_.data_ptr(), stream),
                      "decode silu_and_mul");
        }
        Ly.down->forward_fp16_bf16(dec_mid_, dec_h_, stream, ModelStage::Decode);
    }
    if (logits == nullptr) {
        efm_check(efm_decode_norm_lm_head_top1(H, m_.vocab, m_.eps, dec_h_.data_ptr(), dec_res_[1].data_ptr(),
                                               final_norm_.data_ptr(), lm_head_.data_ptr(), token_buf,
                                               top1_ws_.data_ptr(), top1_ws_.nbytes(), stream),
                  "decode lm head top1");
    } else {
        efm_check(efm_fused_add_rms_norm(1, (uint32_t)H, m_.eps, dec_h_.data_ptr(), dec_res_[1].data_ptr(),
                                         final_norm_.data_ptr(), stream),
                  "decode final norm");
        efm_check(efm_linear(1, H, m_.vocab, dec_h_.data_ptr(), lm_head_.data_ptr(), nullptr, logits, EFM_DTYPE_F32,
                             stream),
                  "decode lm head");
    }
}

// =================================================================================
// Decode plan
// =================================================================================
DecodeLayerPlan resolve_decode_layer(const EngineConfig& cfg, const ModelConfig& m, int32_t layer,
                                     uint32_t max_kv_len, bool allow_fused_front, LinearLayer& o_proj,
                                     LinearLayer& down) {
    const std::string model = cfg.model_name(), hw = cfg.hw_profile(), table = cfg.operator_table_path();
    DecodeLayerPlan P;
    // attention (AttentionLayer::resolve_impl, attention.cu:211-276)
    AttentionOpContext ctx;
    ctx.num_qo_heads = (uint32_t)m.heads;
    ctx.num_kv_heads = (uint32_t)m.kv_heads;
    ctx.head_dim = (uint32_t)m.head_dim;
    ctx.rope_theta = m.theta;
    ctx.dtype = DType::BFloat16;
    ctx.pos_encoding = m.mrope ? AttentionPosEncoding::kNone : AttentionPosEncoding::kRoPELlama;
    ctx.device_id = cfg.device_id();
    ctx.decode_hidden = allow_fused_front ? (uint32_t)m.hidden : 0;   // the fused launch needs it
    ctx.decode_max_kv_len = max_kv_len;
    OperatorQuery q;
    q.op_kind = "attention";
    q.op_name = "attention";
    q.stage = "decode";
    q.shape_sig = attention_shape_sig(ctx.num_qo_heads, ctx.num_kv_heads, ctx.head_dim);
    AttentionOp* attn = nullptr;
    if (auto rec = OperatorImplTable::instance().resolve(model, hw, table, q)) {
        attn = AttentionOpRegistry::instance().find_impl_by_id(rec->impl_id);
        if (attn == nullptr)
            throw ConfigurationError("AttentionLayer: operator_impl_table selected unknown impl '" + rec->impl_id + "'");
        ctx.impl_params = rec->impl_params;
        if (!attn->supports(ctx)) attn = nullptr;   // registry default instead (attention.cu:257-273)
    }
    if (attn == nullptr) attn = AttentionOpRegistry::instance().default_impl(ctx);
    P.attention = attn->impl_id();
    // o_proj, and whether the split partials merge in its prologue
    P.o_proj = o_proj.selected_impl_id(ModelStage::Decode, 1);
    const bool merge = P.o_proj == "hip_gfx950_decode_merge_o_proj";
    if (P.attention == "hip_gfx950_decode_fused_qkv_attention" && !merge)
        throw ConfigurationError("decode layer " + std::to_string(layer) + ": attention impl '" + P.attention +
                                 "' leaves split partials, which o_proj impl '" + P.o_proj + "' cannot merge");
    P.partials_to_o_proj = merge && P.attention != "hip_gfx950_attention";
    // gate/up with the post-attention norm and SwiGLU fused (try_forward_decode_swiglu_fused,
    // linear.cu:2054-2201: unknown or unsupporting record -> ConfigurationError), else,
    // when no impl supports the shape, the layered MLP
    FusedGateUpActivationContext g;
    g.stage = ModelStage::Decode;
    g.m = 1;
    g.hidden = m.hidden;
    g.intermediate = m.inter;
    OperatorQuery gq;
    gq.op_kind = "fused_gate_up_activation";
    gq.layer_role = "fused_gate_up";
    gq.op_name = "model.layers." + std::to_string(layer) + ".mlp";
    gq.stage = "decode";
    LinearLayer::LinearShapeSignature gs;
    gs.m = 1;
    gs.in_features = (uint32_t)m.hidden;
    gs.out_features = 2 * (uint32_t)m.inter;
    gq.shape_sig = gs.to_string();
    FusedGateUpActivationOp* gop = nullptr;
    if (auto rec = OperatorImplTable::instance().resolve(model, hw, table, gq)) {
        gop = FusedGateUpActivationRegistry::instance().find_impl_by_id(rec->impl_id);
        if (gop == nullptr)
            throw ConfigurationError("FusedGateUpLinearLayer: operator_impl_table selected unknown impl '" +
                                     rec->impl_id + "'");
        if (!gop->supports(g))
            throw ConfigurationError("FusedGateUpLinearLayer: operator_impl_table selected unsupported impl '" +
                                     rec->impl_id + "'");
    } else {
        gop = FusedGateUpActivationRegistry::instance().default_impl(g);
    }
    P.gate_up = gop ? gop->impl_id() : "";
    P.down = down.selected_impl_id(ModelStage::Decode, 1);
    return P;
}

std::vector<DecodeLayerPlan> plan_decode(const std::string& engine_config_path, uint32_t max_kv_len) {
    EngineConfig cfg(engine_config_path);
    const ModelConfig m = ModelConfig::from_json(cfg.model_config());
    std::vector<DecodeLayerPlan> out;
    for (int l = 0; l < m.layers; ++l) {
        const std::string p = "model.layers." + std::to_string(l) + ".";
        LinearLayer o(p + "self_attn.o_proj", cfg, (uint32_t)m.q_dim(), (uint32_t)m.hidden);
        LinearLayer d(p + "mlp.down_proj", cfg, (uint32_t)m.inter, (uint32_t)m.hidden);
        out.push_back(resolve_decode_layer(cfg, m, l, max_kv_len, cfg.decode_fused_qkv_attention() && !m.mrope, o, d));
    }
    return out;
}

// =================================================================================
// StandardEngine
// =================================================================================
namespace {
struct EventTimer {
    hipEvent_t a = nullptr, b = nullptr;
    EventTimer() {
        hip_check(hipEventCreate(&a), "event");
        hip_check(hipEventCreate(&b), "event");
    }
    ~EventTimer() {
        hipEventDestroy(a);
        hipEventDestroy(b);
    }
    double ms() { return between(a, b); }
    static double between(hipEvent_t x, hipEvent_t y) {
        float t = 0.f;
        hip_check(hipEventElapsedTime(&t, x, y), "event elapsed");
        return t;
    }
};

// Per-stage GPU time of the eager decode loop: events recorded between the model, the
// sampler and the finalize of every step, summed after the loop's one synchronisation
// (the reference's GenerateMetricsAccum, standard_engine.cpp:420-460).
struct StageEvents {
    std::vector<hipEvent_t> ev;
    ~StageEvents() {
        for (hipEvent_t e : ev) hipEventDestroy(e);
    }
    hipEvent_t record(hipStream_t s) {
        hipEvent_t e = nullptr;
        hip_check(hipEventCreate(&e), "event");
        ev.push_back(e);
        hip_check(hipEventRecord(e, s), "event");
        return e;
    }
};

double host_ms_since(std::chrono::steady_clock::time_point t0) {
    return std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t0).count();
}
}  // namespace

StandardEngine::StandardEngine(const std::string& config_path) : cfg_(config_path), compact_vocab_(cfg_) {
    // sampling parameters are validated before any device work (src/layers/sampler.cu:130-132)
    check<ConfigurationError>(cfg_.temperature() >= 0.0f,
                              "temperature must be non-negative. Got: " + std::to_string(cfg_.temperature()));
    check<ConfigurationError>(cfg_.top_p() > 0.0f, "top_p must be positive. Got: " + std::to_string(cfg_.top_p()));
    device_id_ = cfg_.device_id();
    hip_check(hipSetDevice(device_id_), "hipSetDevice");
    hip_check(hipStreamCreateWithFlags(&stream_, hipStreamNonBlocking), "hipStreamCreate");
    const ModelConfig m = ModelConfig::from_json(cfg_.model_config());
    auto& loader = WeightLoader::instance();
    if (!loader.has_stage(ModelStage::Prefill)) {
        loader.load_weights_from_file(cfg_.prefill_model_path(), ModelStage::Prefill, device_id_,
                                      cfg_.model_name() == "qwen2_5_vl");
    }
    model_ = std::make_unique<Qwen2_5>(cfg_, m, loader.get(ModelStage::Prefill), device_id_);
    // fixed KV prefixes are configuration ids: remapped like EOS ids (kv_manager.cpp:151-155)
    std::vector<KVSlotConfig> slots = cfg_.kv_slots();
    for (auto& s : slots)
        s.prefix_token_ids = compact_vocab_.remap_required_token_ids(s.prefix_token_ids,
                                                                     "kvcache.requests[].prefix_token_ids");
    kv_ = std::make_unique<KVManager>(slots, m, device_id_);
    state_ = Tensor::zeros({16}, DType::Int32, Device::GPU, device_id_);
    int32_t max_resp = 1;
    for (const auto& s : cfg_.kv_slots()) {
        max_resp = std::max(max_resp, s.max_tokens + 1);
        model_->reserve_decode((uint32_t)s.max_tokens);
    }
    response_dev_ = Tensor::zeros({(int64_t)max_resp}, DType::Int32, Device::GPU, device_id_);
    logits_ = Tensor::zeros({m.vocab}, DType::Float32, Device::GPU, device_id_);
    // per-token logits record: one row per response slot, allocated once so that captured
    // decode graphs keep a valid destination
    if (cfg_.debug_logits())
        logits_hist_ = Tensor::zeros({(int64_t)max_resp, m.vocab}, DType::Float32, Device::GPU, device_id_);
    sample_ws_ = Tensor::zeros({(int64_t)std::max(efm_sampler_greedy_workspace_bytes(1, m.vocab),
                                                   efm_sampler_top_p_workspace_bytes(m.vocab))},
                               DType::UInt8, Device::GPU, device_id_);
    warmup();
}

StandardEngine::~StandardEngine() {
    drop_graphs();
    drop_prefill_graphs();
    if (stream_) hipStreamDestroy(stream_);
}

void StandardEngine::drop_prefill_graphs() {
    for (auto& kv : pf_graphs_) {
        if (kv.second.exec) hipGraphExecDestroy(kv.second.exec);
        if (kv.second.graph) hipGraphDestroy(kv.second.graph);
    }
    pf_graphs_.clear();
}

uint64_t StandardEngine::prefill_epoch() const { return pf_input_epoch_ + model_->prefill_buffers_epoch(); }

void StandardEngine::drop_graphs() {
    for (auto& kv : graphs_) {
        if (kv.second.exec) hipGraphExecDestroy(kv.second.exec);
        if (kv.second.graph) hipGraphDestroy(kv.second.graph);
        if (kv.second.exec_n) hipGraphExecDestroy(kv.second.exec_n);
        if (kv.second.graph_n) hipGraphDestroy(kv.second.graph_n);
    }
    graphs_.clear();
}

std::vector<void*> StandardEngine::caches(int32_t request_id, bool k) {
    std::vector<void*> out;
    for (int l = 0; l < model_->config().layers; ++l)
        out.push_back(k ? kv_->k_cache(request_id, l) : kv_->v_cache(request_id, l));
    return out;
}

// Fixed-prefix KV: prefill every slot's prefix once (standard_engine.cpp:515-556).
void StandardEngine::warmup() {
    for (int32_t rid : kv_->request_ids()) {
        KVSlot& s = kv_->slot(rid);
        if (s.prefix_size == 0 || s.prefix_ready) continue;
        const int32_t n = s.prefix_size;
        if (ids_dev_.empty() || ids_dev_.numel() < n) {
            ids_dev_ = Tensor::empty({n}, DType::Int32, Device::GPU, device_id_);
            ++pf_input_epoch_;
        }
        hip_check(hipMemcpyAsync(ids_dev_.data_ptr(), s.cfg.prefix_token_ids.data(), (size_t)n * 4,
                                 hipMemcpyHostToDevice, stream_),
                  "prefix ids");
        auto kc = caches(rid, true), vc = caches(rid, false);
        int32_t* tok = static_cast<int32_t*>(state_.data_ptr()) + 2;
        model_->prefill(n, 0, static_cast<int32_t*>(ids_dev_.data_ptr()), nullptr, -1, nullptr, kc.data(), vc.data(),
                        tok, nullptr, stream_);
        hip_check(hipStreamSynchronize(stream_), "prefix warmup");
        s.prefix_ready = true;
    }
}

void StandardEngine::sample_logits(uint32_t) {
    int32_t* tok = static_cast<int32_t*>(state_.data_ptr()) + 2;
    const float T = cfg_.temperature();
    if (!logits_hist_.empty()) {
        // row = response index of the token about to be sampled (device step counter)
        const int64_t V = model_->config().vocab;
        efm_check(efm_store_row_indexed(logits_.data_ptr(), logits_hist_.data_ptr(), V * 4,
                                        static_cast<const uint32_t*>(state_.data_ptr()) + 1,
                                        (uint32_t)logits_hist_.shape()[0], stream_),
                  "logits record");
    }
    if (T < 1e-6f) {
        efm_check(efm_sampler_greedy(1, model_->config().vocab, static_cast<float*>(logits_.data_ptr()), tok,
                                     sample_ws_.data_ptr(), sample_ws_.nbytes(), stream_),
                  "greedy sampler");
        return;
    }
    // temperature / top-p: the draw's counter is the response index of the token being
    // sampled (device-resident step counter), so graph replays draw fresh numbers
    const int32_t* d_step = static_cast<const int32_t*>(state_.data_ptr()) + 1;
    efm_check(efm_sampler_top_p(model_->config().vocab, static_cast<const float*>(logits_.data_ptr()), T,
                                cfg_.top_p(), cfg_.seed(), 0, d_step, tok, sample_ws_.data_ptr(), sample_ws_.nbytes(),
                                stream_),
              "top-p sampler");
}

uint32_t StandardEngine::decode_row_bound(uint32_t rows, uint32_t capacity) {
    const uint32_t b = (std::max<uint32_t>(rows, 1u) + kDecodeBoundRows - 1) / kDecodeBoundRows * kDecodeBoundRows;
    return std::min(b, capacity);
}

void StandardEngine::run_decode_step(int32_t request_id, void* stage_events, uint32_t row_bound) {
    StageEvents* se = static_cast<StageEvents*>(stage_events);
    int32_t* st = static_cast<int32_t*>(state_.data_ptr());
    uint32_t* d_kv_len = reinterpret_cast<uint32_t*>(st + 0);
    uint32_t* d_step = reinterpret_cast<uint32_t*>(st + 1);
    int32_t* tok = st + 2;
    const int32_t* pos3 = st + 3;
    KVSlot& slot = kv_->slot(request_id);
    auto kc = caches(request_id, true), vc = caches(request_id, false);
    const bool greedy_fused = cfg_.temperature() < 1e-6f && cfg_.lm_head_top1() && !cfg_.debug_logits();
    if (se) se->record(stream_);
    {
        RoctxRange r(se ? "EDGEFM_DECODE_MODEL" : nullptr);
        check<InternalError>(row_bound >= 1 && row_bound <= (uint32_t)slot.cfg.max_tokens, "decode row bound");
        model_->decode_step(tok, d_kv_len, row_bound, pos3, kc.data(), vc.data(),
                            greedy_fused ? nullptr : static_cast<float*>(logits_.data_ptr()), stream_);
    }
    if (se) se->record(stream_);
    if (!greedy_fused) {
        RoctxRange r(se ? "EDGEFM_DECODE_SAMPLER" : nullptr);
        sample_logits(0);
    }
    if (se) se->record(stream_);
    efm_check(efm_finalize_decode_token_indexed(tok, static_cast<int32_t*>(response_dev_.data_ptr()), d_step, d_kv_len,
                                                (uint32_t)response_dev_.numel(), stream_),
              "finalize decode token");
    if (model_->config().mrope) efm_check(efm_increment_int32_triplet(st + 3, stream_), "advance mrope position");
    if (se) se->record(stream_);
}

Response StandardEngine::generate(const Request& request) {
    RoctxRange generate_range("EDGEFM_GENERATE");
    hip_check(hipSetDevice(device_id_), "hipSetDevice");
    const auto prep_t0 = std::chrono::steady_clock::now();
    std::optional<RoctxRange> prepare_range(std::in_place, "EDGEFM_PREFILL_PREPARE");
    // compact vocabulary: the request is remapped into the checkpoint's ids and the
    // response restored (standard_engine.cpp:877-882,1070-1072)
    std::unique_ptr<Request> remapped;
    if (compact_vocab_.enabled()) remapped = std::make_unique<Request>(compact_vocab_.remap_request(request));
    const Request& req = remapped ? *remapped : request;
    check<InvalidRequestError>(!req.token_ids.empty(), "Request must contain at least one token id");
    KVSlot& slot = kv_->slot(req.request_id);
    const ModelConfig& m = model_->config();
    const int32_t n_ids = (int32_t)req.token_ids.size();
    check<InvalidRequestError>(n_ids <= slot.cfg.max_tokens, "Request sequence length exceeds kvcache max_tokens");
    for (int32_t id : req.token_ids) {
        const bool custom = req.has_embedding() && req.embed_token_id >= 0 && id >= req.embed_token_id &&
                            id < req.embed_token_id + req.embedding.shape()[0];
        check<InvalidRequestError>(custom || (id >= 0 && id < m.vocab), "token id out of vocabulary range");
    }
    if (m.mrope) check<InvalidRequestError>(req.has_position_ids(), "Qwen2.5-VL requests need position_ids [3, S]");

    // prefix handling: ids starting with the slot prefix only prefill the suffix
    // (standard_engine.cpp:1213-1235)
    int32_t base = 0;
    if (slot.prefix_size > 0 && n_ids > slot.prefix_size &&
        std::equal(slot.cfg.prefix_token_ids.begin(), slot.cfg.prefix_token_ids.end(), req.token_ids.begin())) {
        // a request that did not start with the prefix overwrote its rows: restore them first
        if (!slot.prefix_ready) warmup();
        base = slot.prefix_size;
    } else if (slot.prefix_size > 0) {
        // this prefill writes rows [0, n_ids) over the stored prefix
        slot.prefix_ready = false;
    }
    const int32_t S = n_ids - base;
    // max_generated = min(max_new_tokens, max_tokens - len(ids) + 1) (scheduler.cpp:123-134)
    const int32_t n_gen = std::max(1, std::min(cfg_.max_new_tokens(), slot.cfg.max_tokens - n_ids + 1));

    if (ids_dev_.empty() || ids_dev_.numel() < S) {
        ids_dev_ = Tensor::empty({S}, DType::Int32, Device::GPU, device_id_);
        ++pf_input_epoch_;
    }
    hip_check(hipMemcpyAsync(ids_dev_.data_ptr(), req.token_ids.data() + base, (size_t)S * 4, hipMemcpyHostToDevice,
                             stream_),
              "token ids H2D");
    Tensor emb, pos;
    if (req.has_embedding()) {
        auto [dev, did] = req.embedding.device();
        emb = (dev == Device::GPU) ? req.embedding
                                   : Tensor::clone_from(req.embedding.data_ptr(), req.embedding.shape(),
                                                        req.embedding.dtype(), Device::CPU, 0, Device::GPU, device_id_,
                                                        stream_);
        check<InvalidRequestError>(emb.dtype() == DType::BFloat16 && emb.shape().size() == 2 &&
                                       emb.shape()[1] == m.hidden,
                                   "embedding must be bf16 [rows, hidden]");
    }
    std::vector<int32_t> last_pos(3, 0);
    if (m.mrope) {
        const auto& ps = req.position_ids.shape();
        check<InvalidRequestError>(ps.size() == 2 && ps[0] == 3 && ps[1] == n_ids && req.position_ids.dtype() == DType::Int32,
                                   "position_ids must be int32 [3, len(token_ids)]");
        std::vector<int32_t> host(3 * (size_t)n_ids);
        auto [dev, did] = req.position_ids.device();
        hip_check(hipMemcpy(host.data(), req.position_ids.data_ptr(), host.size() * 4,
                            dev == Device::GPU ? hipMemcpyDeviceToHost : hipMemcpyHostToHost),
                  "position ids");
        // positions of the prefilled rows [base, n_ids)
        std::vector<int32_t> sub(3 * (size_t)S);
        for (int r = 0; r < 3; ++r)
            std::copy(host.begin() + (size_t)r * n_ids + base, host.begin() + (size_t)(r + 1) * n_ids,
                      sub.begin() + (size_t)r * S);
        pos = Tensor::clone_from(sub.data(), {3, S}, DType::Int32, Device::CPU, 0, Device::GPU, device_id_, stream_);
        // decode positions continue from the request's last position triplet, or the
        // global max replicated (src/models/model.cpp:34-45; +1 for hidden >= 3584,
        // qwen2_5.cpp:974-978)
        if (req.mrope_last_pos.size() == 3) {
            last_pos = req.mrope_last_pos;
        } else {
            const int32_t mx = *std::max_element(host.begin(), host.end());
            last_pos = {mx, mx, mx};
            if (m.hidden >= 3584)
                for (auto& p : last_pos) p += 1;
        }
    }

    metrics_.clear();
    EventTimer pf, dc;
    auto kc = caches(req.request_id, true), vc = caches(req.request_id, false);
    int32_t* st = static_cast<int32_t*>(state_.data_ptr());
    // decode state: d_kv_len = rows after prefill, step = 0, positions = last + 1
    int32_t init[6] = {base + S, 0, 0, last_pos[0] + 1, last_pos[1] + 1, last_pos[2] + 1};
    hip_check(hipMemcpyAsync(st, init, sizeof(init), hipMemcpyHostToDevice, stream_), "decode state H2D");

    const double prefill_prepare_host_ms = host_ms_since(prep_t0);
    prepare_range.reset();

    EventTimer pf_model;  // pf.a .. pf_model.b: model; pf_model.b .. pf.b: sampler + finalize
    const bool greedy_fused = cfg_.temperature() < 1e-6f && cfg_.lm_head_top1() && !cfg_.debug_logits();
    // graph mode: custom embeddings and M-RoPE positions go to persistent buffers that a
    // captured prefill reads (stream-ordered copies ahead of the replay)
    if (cfg_.use_graph()) {
        if (!emb.empty()) {
            if (pf_emb_dev_.empty() || pf_emb_dev_.nbytes() < emb.nbytes()) {
                pf_emb_dev_ = Tensor::empty({(int64_t)emb.numel()}, DType::BFloat16, Device::GPU, device_id_);
                ++pf_input_epoch_;
            }
            hip_check(hipMemcpyAsync(pf_emb_dev_.data_ptr(), emb.data_ptr(), emb.nbytes(), hipMemcpyDeviceToDevice,
                                     stream_),
                      "stage embeddings");
            emb = pf_emb_dev_.prefix_view(emb.shape());
        }
        if (!pos.empty()) {
            if (pf_pos_dev_.empty() || pf_pos_dev_.nbytes() < pos.nbytes()) {
                pf_pos_dev_ = Tensor::empty({(int64_t)pos.numel()}, DType::Int32, Device::GPU, device_id_);
                ++pf_input_epoch_;
            }
            hip_check(hipMemcpyAsync(pf_pos_dev_.data_ptr(), pos.data_ptr(), pos.nbytes(), hipMemcpyDeviceToDevice,
                                     stream_),
                      "stage position ids");
            pos = pf_pos_dev_.prefix_view(pos.shape());
        }
    }
    auto prefill_work = [&]() {
        model_->prefill(S, base, static_cast<int32_t*>(ids_dev_.data_ptr()), emb.empty() ? nullptr : &emb,
                        req.embed_token_id, pos.empty() ? nullptr : static_cast<int32_t*>(pos.data_ptr()), kc.data(),
                        vc.data(), st + 2, greedy_fused ? nullptr : static_cast<float*>(logits_.data_ptr()), stream_);
    };
    auto finalize_work = [&]() {
        if (!greedy_fused) sample_logits(0);
        efm_check(efm_finalize_decode_token_indexed(st + 2, static_cast<int32_t*>(response_dev_.data_ptr()),
                                                    reinterpret_cast<uint32_t*>(st + 1),
                                                    reinterpret_cast<uint32_t*>(st), (uint32_t)response_dev_.numel(),
                                                    stream_),
                  "finalize prefill token");
    };
    bool prefill_replayed = false;
    if (cfg_.use_graph()) {
        const PrefillKey key{req.request_id, S, base, emb.empty() ? 0 : emb.shape()[0],
                             emb.empty() ? -1 : req.embed_token_id};
        const uint64_t epoch = prefill_epoch();
        auto it = pf_graphs_.find(key);
        if (it != pf_graphs_.end() && it->second.epoch != epoch) {
            hipGraphExecDestroy(it->second.exec);
            hipGraphDestroy(it->second.graph);
            pf_graphs_.erase(it);
            it = pf_graphs_.end();
        }
        if (it == pf_graphs_.end() && pf_seen_.count(key)) {
            if (pf_graphs_.size() >= kMaxPrefillGraphs) drop_prefill_graphs();
            RoctxRange capture_range("EDGEFM_PREFILL_CAPTURE");
            PrefillGraph g;
            hip_check(hipStreamBeginCapture(stream_, hipStreamCaptureModeThreadLocal), "begin prefill capture");
            try {
                prefill_work();
                finalize_work();
            } catch (...) {
                hipGraph_t tmp = nullptr;
                hipStreamEndCapture(stream_, &tmp);
                if (tmp) hipGraphDestroy(tmp);
                throw;
            }
            hip_check(hipStreamEndCapture(stream_, &g.graph), "end prefill capture");
            hip_check(hipGraphInstantiate(&g.exec, g.graph, nullptr, nullptr, 0), "prefill graph instantiate");
            g.epoch = epoch;
            it = pf_graphs_.emplace(key, g).first;
        }
        if (it != pf_graphs_.end()) {
            RoctxRange replay_range("EDGEFM_PREFILL_GRAPH_REPLAY");
            hip_check(hipEventRecord(pf.a, stream_), "event");
            hip_check(hipGraphLaunch(it->second.exec, stream_), "prefill graph launch");
            hip_check(hipEventRecord(pf_model.b, stream_), "event");
            prefill_replayed = true;
        } else {
            pf_seen_.insert(key);
        }
    }
    if (!prefill_replayed) {
        hip_check(hipEventRecord(pf.a, stream_), "event");
        RoctxRange prefill_range("EDGEFM_PREFILL");
        {
            RoctxRange model_range("EDGEFM_PREFILL_MODEL");
            prefill_work();
        }
        hip_check(hipEventRecord(pf_model.b, stream_), "event");
        RoctxRange sampler_range("EDGEFM_PREFILL_SAMPLER");
        finalize_work();
    }
    hip_check(hipEventRecord(pf.b, stream_), "event");

    const auto dprep_t0 = std::chrono::steady_clock::now();
    double decode_prepare_host_ms = 0.0;
    StageEvents stage;
    hip_check(hipEventRecord(dc.a, stream_), "event");
    const int32_t steps = n_gen - 1;
    if (steps > 0) {
        RoctxRange decode_range("EDGEFM_GENERATION");
        // decode step i attends base + S + i + 1 rows; its launches read below a 128-row bound:
        // that of the last step of its kGraphSteps group (a graph's steps share one bound), or
        // its own past the last whole group. Eager decoding uses the same bounds, so both
        // run the same kernels.
        const uint32_t cap = (uint32_t)slot.cfg.max_tokens;
        auto bound_at = [&](int32_t step_end) { return decode_row_bound((uint32_t)(base + S + step_end), cap); };
        const int32_t grouped = steps / kGraphSteps * kGraphSteps;
        auto step_bound = [&](int32_t i) {
            return i < grouped ? bound_at((i / kGraphSteps + 1) * kGraphSteps) : bound_at(i + 1);
        };
        if (cfg_.use_graph()) {
            // every step reads its position and writes its token through device state, so
            // n consecutive captures of one step replay as n steps
            auto capture = [&](int32_t n, uint32_t bound, hipGraph_t* graph, hipGraphExec_t* exec) {
                RoctxRange capture_range("EDGEFM_DECODE_PREPARE");
                model_->reserve_decode(bound);
                hip_check(hipStreamBeginCapture(stream_, hipStreamCaptureModeThreadLocal), "begin capture");
                try {
                    for (int32_t i = 0; i < n; ++i) run_decode_step(req.request_id, nullptr, bound);
                } catch (...) {
                    hipGraph_t tmp = nullptr;
                    hipStreamEndCapture(stream_, &tmp);
                    if (tmp) hipGraphDestroy(tmp);
                    throw;
                }
                hip_check(hipStreamEndCapture(stream_, graph), "end capture");
                hip_check(hipGraphInstantiate(exec, *graph, nullptr, nullptr, 0), "graph instantiate");
            };
            // the launch sequence (graph of kGraphSteps steps or of one, and its bound); every
            // graph it needs is captured before the first replay
            std::vector<std::pair<hipGraphExec_t*, uint32_t>> seq;
            int32_t done = 0;
            for (; done + kGraphSteps <= steps; done += kGraphSteps) {
                const uint32_t bound = step_bound(done);
                GraphEntry& g = graphs_[{req.request_id, bound}];
                if (g.exec_n == nullptr) capture(kGraphSteps, bound, &g.graph_n, &g.exec_n);
                seq.push_back({&g.exec_n, bound});
            }
            for (; done < steps; ++done) {
                const uint32_t bound = step_bound(done);
                GraphEntry& g = graphs_[{req.request_id, bound}];
                if (g.exec == nullptr) capture(1, bound, &g.graph, &g.exec);
                seq.push_back({&g.exec, bound});
            }
            decode_prepare_host_ms = host_ms_since(dprep_t0);
            RoctxRange replay_range("EDGEFM_DECODE_GRAPH_REPLAY");
            for (const auto& e : seq) hip_check(hipGraphLaunch(*e.first, stream_), "graph launch");
        } else {
            for (int32_t i = 0; i < steps; ++i) {
                const uint32_t bound = step_bound(i);
                model_->reserve_decode(bound);
                run_decode_step(req.request_id, &stage, bound);
            }
        }
    }
    hip_check(hipEventRecord(dc.b, stream_), "event");

    last_n_gen_ = n_gen;
    std::vector<int32_t> host((size_t)n_gen);
    EventTimer copy;
    {
        RoctxRange copy_range("EDGEFM_RESPONSE_COPY");
        hip_check(hipEventRecord(copy.a, stream_), "event");
        hip_check(hipMemcpyAsync(host.data(), response_dev_.data_ptr(), (size_t)n_gen * 4, hipMemcpyDeviceToHost,
                                 stream_),
                  "response D2H");
        hip_check(hipEventRecord(copy.b, stream_), "event");
        hip_check(hipStreamSynchronize(stream_), "generate sync");
    }
    try {
        model_->check_decode_status(stream_);
    } catch (const DeviceError&) {
        // A decode launch gave up a bounded wait: this response is wrong and is not
        // returned. The launches' device state is already reset; the captured decode
        // graphs are dropped as well, so the next call captures its launches afresh.
        drop_graphs();
        throw;
    }

    // stop tokens truncate after the first hit, inclusive (standard_engine.cpp:1060-1068)
    const auto stop_t0 = std::chrono::steady_clock::now();
    if (!req.ignore_stop_tokens) {
        std::unordered_set<int32_t> stop;
        for (int32_t t : compact_vocab_.remap_required_token_ids(cfg_.eos_token_ids(), "model eos_token_ids"))
            stop.insert(t);
        for (int32_t t : compact_vocab_.remap_required_token_ids(cfg_.stop_token_ids(), "sampling.stop_token_ids"))
            stop.insert(t);
        for (int32_t t : req.stop_token_ids) stop.insert(t);
        for (size_t i = 0; i < host.size(); ++i)
            if (stop.count(host[i])) {
                host.resize(i + 1);
                break;
            }
    }
    const double stop_check_host_ms = host_ms_since(stop_t0);
    const double prefill_ms = pf.ms(), decode_ms = dc.ms();
    // eager decode: per-step model / sampler / finalize spans (four events per step)
    double d_model = 0.0, d_sampler = 0.0, d_finalize = 0.0;
    for (size_t i = 0; i + 3 < stage.ev.size(); i += 4) {
        d_model += EventTimer::between(stage.ev[i], stage.ev[i + 1]);
        d_sampler += EventTimer::between(stage.ev[i + 1], stage.ev[i + 2]);
        d_finalize += EventTimer::between(stage.ev[i + 2], stage.ev[i + 3]);
    }
    const bool graph = cfg_.use_graph() && steps > 0;
    const double returned = (double)host.size();
    const double returned_steps = std::max(0.0, returned - 1.0);
    // the reference's keys (standard_engine.cpp:462-507), then this engine's own
    metrics_["prefill_ms"] = prefill_ms;
    metrics_["decode_ms"] = decode_ms;
    metrics_["total_stage_ms"] = prefill_ms + decode_ms;
    metrics_["decode_step_avg_ms"] = steps > 0 ? decode_ms / steps : 0.0;
    metrics_["generated_tokens_total"] = returned;
    metrics_["decode_steps"] = steps;
    metrics_["prefill_prepare_host_ms"] = prefill_prepare_host_ms;
    metrics_["prefill_model_ms"] = EventTimer::between(pf.a, pf_model.b);
    metrics_["prefill_sampler_ms"] = EventTimer::between(pf_model.b, pf.b);
    metrics_["decode_prepare_host_ms"] = decode_prepare_host_ms;
    metrics_["decode_graph_replay_ms"] = graph ? decode_ms : 0.0;
    metrics_["decode_model_ms"] = d_model;
    metrics_["decode_sampler_ms"] = d_sampler;
    metrics_["decode_finalize_ms"] = d_finalize;
    metrics_["stop_check_host_ms"] = stop_check_host_ms;
    metrics_["response_copy_ms"] = copy.ms();
    metrics_["tokens_per_second"] = (prefill_ms + decode_ms) > 0 ? returned * 1000.0 / (prefill_ms + decode_ms) : 0.0;
    metrics_["decode_tokens_per_second"] = decode_ms > 0 ? returned_steps * 1000.0 / decode_ms : 0.0;
    metrics_["executed_generated_tokens_total"] = n_gen;
    metrics_["returned_generated_tokens_total"] = returned;
    metrics_["cuda_graph_enabled"] = cfg_.use_graph() ? 1.0 : 0.0;
    metrics_["prefill_graph_replayed"] = prefill_replayed ? 1.0 : 0.0;
    metrics_["lm_head_top1_enabled"] = greedy_fused ? 1.0 : 0.0;
    metrics_["lm_head_top1_decode_steps"] = greedy_fused ? steps : 0.0;
    metrics_["response_tokens_capacity"] = (double)response_dev_.numel();
    metrics_["prefill_tokens"] = S;
    metrics_["prefill_tokens_per_second"] = prefill_ms > 0 ? S * 1000.0 / prefill_ms : 0.0;
    metrics_["decode_fused_qkv_attention"] = model_->uses_fused_front((uint32_t)slot.cfg.max_tokens) ? 1.0 : 0.0;
    Response r;
    r.token_ids = compact_vocab_.restore_token_ids(host, "response token_ids");
    return r;
}

EdgeFM::EdgeFM(const std::string& config_path) : engine_(std::make_unique<StandardEngine>(config_path)) {}
Response EdgeFM::generate(const Request& request) const { return engine_->generate(request); }
std::vector<float> EdgeFM::last_logits(int32_t* rows, int32_t* vocab) const { return engine_->last_logits(rows, vocab); }

std::vector<float> StandardEngine::last_logits(int32_t* rows, int32_t* vocab) const {
    if (logits_hist_.empty())
        throw ConfigurationError("EdgeFM.last_logits: the engine config does not set runtime.debug_logits");
    const int64_t V = model_->config().vocab;
    const int32_t n = std::min<int32_t>(last_n_gen_, (int32_t)logits_hist_.shape()[0]);
    std::vector<float> out((size_t)n * (size_t)V);
    if (n > 0)
        hip_check(hipMemcpy(out.data(), logits_hist_.data_ptr(), out.size() * sizeof(float), hipMemcpyDeviceToHost),
                  "logits record D2H");
    *rows = n;
    *vocab = (int32_t)V;
    return out;
}
std::unordered_map<std::string, double> EdgeFM::last_generate_metrics() const { return engine_->last_generate_metrics(); }

}  // namespace edge_fm
