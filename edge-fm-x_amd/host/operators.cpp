#include "operators.hpp"

#include <cctype>
#include <filesystem>
#include <map>
#include <mutex>

namespace edge_fm {

// ---------------------------------------------------------------------------------
// Operator implementation table
// ---------------------------------------------------------------------------------
std::string normalize_identifier(const std::string& raw) {
    std::string out;
    out.reserve(raw.size());
    for (unsigned char c : raw) {
        if (std::isalnum(c)) out.push_back((char)std::tolower(c));
        else if (c == '_' || c == '.' || c == '-' || c == ' ' || c == '/' || c == ':') out.push_back('_');
    }
    return out;
}

std::string normalize_model_name(const std::string& raw) {
    const std::string n = normalize_identifier(raw);
    if (n == "qwen2_5" || n == "qwen25" || n == "qwen2") return "qwen2_5";
    if (n == "qwen2_5_vl" || n == "qwen25_vl" || n == "qwen2_vl" || n == "qwen25vl" || n == "qwen2_5vl" ||
        n == "qwen2vl")
        return "qwen2_5_vl";
    return n;
}

Json OperatorImplRecord::to_json() const {
    Json j = Json::object();
    j["model_name"] = model_name;
    j["hw_profile"] = hw_profile;
    j["op_kind"] = op_kind;
    j["layer_role"] = layer_role;
    j["op_name"] = op_name;
    j["stage"] = stage;
    j["shape_sig"] = shape_sig;
    j["impl_id"] = impl_id;
    j["impl_params"] = impl_params;
    return j;
}

OperatorImplRecord OperatorImplRecord::from_json(const Json& j) {
    OperatorImplRecord r;
    r.model_name = normalize_model_name(j.get_string("model_name"));
    r.hw_profile = normalize_identifier(j.get_string("hw_profile"));
    r.op_kind = normalize_identifier(j.get_string("op_kind"));
    r.layer_role = normalize_identifier(j.get_string("layer_role"));
    r.op_name = normalize_identifier(j.get_string("op_name"));
    r.stage = normalize_identifier(j.get_string("stage"));
    r.shape_sig = j.get_string("shape_sig");
    r.impl_id = j.get_string("impl_id");
    if (r.impl_id.empty()) throw ConfigurationError("operator_impl_table record without impl_id");
    if (j.contains("impl_params") && j.at("impl_params").is_object()) r.impl_params = j.at("impl_params");
    return r;
}

static std::vector<OperatorImplRecord> builtin_records() {
    std::vector<OperatorImplRecord> out;
    const char* kinds[][2] = {{"linear", "hip_gfx950_linear"},
                              {"attention", "hip_gfx950_attention"},
                              {"norm", "hip_gfx950_norm"},
                              {"activation", "hip_gfx950_silu_and_mul"},
                              {"fused_gate_up_activation", "hip_gfx950_swiglu"}};
    for (const char* model : {"qwen2_5", "qwen2_5_vl"}) {
        for (auto& k : kinds) {
            OperatorImplRecord r;
            r.model_name = model;
            r.hw_profile = "rocm";
            r.op_kind = k[0];
            r.impl_id = k[1];
            out.push_back(r);
        }
    }
    return out;
}

static int match_field(const std::string& pattern, const std::string& query, int exact) {
    if (pattern.empty() || pattern == "*") return 0;
    return pattern == query ? exact : -1;
}

static int match_hw(const std::string& pattern, const std::string& query) {
    if (pattern.empty() || pattern == "*") return 0;
    if (pattern == query) return 200;
    if (query.rfind(pattern + "_", 0) == 0) return 120;
    return -1;
}

OperatorImplTable& OperatorImplTable::instance() {
    static OperatorImplTable t;
    return t;
}

static std::string table_key(const std::string& path) {
    if (path.empty()) return "<builtin>";
    return std::filesystem::absolute(std::filesystem::path(path)).lexically_normal().string();
}

const std::vector<OperatorImplRecord>& OperatorImplTable::load_locked(const std::string& path) {
    const std::string key = table_key(path);
    auto it = tables_.find(key);
    if (it != tables_.end()) return it->second;
    std::vector<OperatorImplRecord> recs = builtin_records();
    if (!path.empty()) {
        Json j;
        try {
            j = Json::parse_file(path);
        } catch (const std::exception& e) {
            throw ConfigurationError("Cannot load operator_impl_table " + path + ": " + e.what());
        }
        if (!j.contains("records") || !j.at("records").is_array())
            throw ConfigurationError("operator_impl_table must contain a records array: " + path);
        for (const auto& r : j.at("records").as_array()) recs.push_back(OperatorImplRecord::from_json(r));
    }
    return tables_.emplace(key, std::move(recs)).first->second;
}

std::optional<OperatorImplRecord> OperatorImplTable::resolve(const std::string& model_name,
                                                             const std::string& hw_profile,
                                                             const std::string& table_path, const OperatorQuery& q) {
    const std::string model = normalize_model_name(model_name);
    const std::string hw = normalize_identifier(hw_profile);
    const std::string kind = normalize_identifier(q.op_kind);
    const std::string role = normalize_identifier(q.layer_role);
    const std::string name = normalize_identifier(q.op_name);
    const std::string stage = normalize_identifier(q.stage);
    std::lock_guard<std::mutex> lock(mu_);
    const auto& recs = load_locked(table_path);
    std::optional<OperatorImplRecord> best;
    int best_score = -1;
    for (const auto& r : recs) {
        const int s_kind = match_field(r.op_kind, kind, 10);
        const int s_model = match_field(r.model_name, model, 100);
        const int s_hw = match_hw(r.hw_profile, hw);
        if (s_kind < 0 || s_model < 0 || s_hw < 0) continue;
        const int s_name = match_field(r.op_name, name, 1000000);
        const int s_role = match_field(r.layer_role, role, 100000);
        const int s_shape = match_field(r.shape_sig, q.shape_sig, 10000);
        const int s_stage = match_field(r.stage, stage, 1000);
        if (s_name < 0 || s_role < 0 || s_shape < 0 || s_stage < 0) continue;
        const int total = s_name + s_role + s_shape + s_stage + s_hw + s_model + s_kind;
        if (total >= best_score) {
            best = r;
            best_score = total;
        }
    }
    return best;
}

std::vector<OperatorImplRecord> OperatorImplTable::all_records(const std::string& table_path) {
    std::lock_guard<std::mutex> lock(mu_);
    return load_locked(table_path);
}

void OperatorImplTable::invalidate(const std::string& table_path) {
    std::lock_guard<std::mutex> lock(mu_);
    tables_.erase(table_key(table_path));
}

std::string resolve_impl_id(const std::string& model_name, const std::string& hw_profile,
                            const std::string& table_path, const OperatorQuery& q, Json* impl_params) {
    auto rec = OperatorImplTable::instance().resolve(model_name, hw_profile, table_path, q);
    if (!rec) return "";
    if (impl_params) *impl_params = rec->impl_params;
    return rec->impl_id;
}

// ---------------------------------------------------------------------------------
// Attention
// ---------------------------------------------------------------------------------
efm_attention_ctx to_c_ctx(const AttentionOpContext& c) {
    efm_attention_ctx r{};
    r.num_qo_heads = c.num_qo_heads;
    r.num_kv_heads = c.num_kv_heads;
    r.head_dim = c.head_dim;
    r.q_stride_n = c.q_stride_n;
    r.q_stride_h = c.q_stride_h;
    r.k_stride_n = c.k_stride_n;
    r.k_stride_h = c.k_stride_h;
    r.kv_stride_n = c.kv_stride_n;
    r.kv_stride_h = c.kv_stride_h;
    r.rope_scale = c.rope_scale;
    r.rope_theta = c.rope_theta;
    r.q_rope_pos_offset = c.q_rope_pos_offset;
    r.k_rope_pos_offset = c.k_rope_pos_offset;
    r.dtype = (int32_t)c.dtype;
    r.pos_encoding = c.pos_encoding == AttentionPosEncoding::kRoPELlama ? EFM_POS_ROPE_LLAMA : EFM_POS_NONE;
    r.k_already_prerotated = c.k_already_prerotated ? 1 : 0;
    return r;
}

namespace {

// Device scratch for split-KV decode partials: grow-only, one per device, reset to zero
// on growth (the kernel leaves its arrival counters at zero after every call). Plays
// the role of StaticBufferManager::get_cache_buf (src/utils/device/memory.h:18-113).
struct DecodeWorkspace {
    std::mutex mu;
    std::unordered_map<int, Tensor> bufs;
    Tensor get(int device, size_t bytes) {
        std::lock_guard<std::mutex> lock(mu);
        auto it = bufs.find(device);
        if (it == bufs.end() || it->second.nbytes() < bytes) {
            bufs[device] = Tensor::zeros({(int64_t)bytes}, DType::UInt8, Device::GPU, device);
        }
        return bufs[device];
    }
};
DecodeWorkspace g_decode_ws;

class HipAttentionOp final : public AttentionOp {
public:
    std::string impl_id() const override { return "hip_gfx950_attention"; }
    bool supports(const AttentionOpContext& c) const override {
        if (c.dtype != DType::BFloat16) return false;
        if (c.head_dim != 64 && c.head_dim != 128) return false;
        if (c.num_kv_heads == 0 || c.num_qo_heads % c.num_kv_heads) return false;
        const uint32_t g = c.num_qo_heads / c.num_kv_heads;
        return g == 1 || g == 2 || g == 3 || g == 4 || g == 6 || g == 7 || g == 8;
    }
    void forward_prefill(const AttentionOpContext& ctx, const Tensor& q, const Tensor& k, const Tensor& v, Tensor& o,
                         bool causal, hipStream_t stream) override {
        check<InvalidRequestError>(!q.shape().empty() && !k.shape().empty(), "attention prefill: empty tensors");
        const efm_attention_ctx c = to_c_ctx(ctx);
        efm_check(efm_attention_prefill(&c, q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(),
                                        (uint32_t)q.shape()[0], (uint32_t)k.shape()[0], causal ? 1 : 0, stream),
                  "attention prefill");
    }
    void forward_decode(const AttentionOpContext& ctx, const Tensor& q, const Tensor& k, const Tensor& v, Tensor& o,
                        hipStream_t stream, uint32_t* d_kv_len, uint32_t max_kv_len) override {
        const efm_attention_ctx c = to_c_ctx(ctx);
        const uint32_t kv_len = (uint32_t)k.shape()[0];
        const uint32_t bound = d_kv_len ? max_kv_len : kv_len;
        const size_t ws_bytes = efm_attention_decode_workspace_bytes(&c, bound);
        Tensor ws = g_decode_ws.get(ctx.device_id, ws_bytes);
        efm_check(efm_attention_decode(&c, q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(), kv_len, d_kv_len,
                                       max_kv_len, ws.data_ptr(), ws.nbytes(), stream),
                  "attention decode");
    }
};

}  // namespace

AttentionOpRegistry::AttentionOpRegistry() { impls_.push_back(std::make_unique<HipAttentionOp>()); }
AttentionOpRegistry& AttentionOpRegistry::instance() {
    static AttentionOpRegistry r;
    return r;
}
AttentionOp* AttentionOpRegistry::find_impl_by_id(const std::string& id) const {
    for (auto& i : impls_)
        if (i->impl_id() == id) return i.get();
    return nullptr;
}
AttentionOp* AttentionOpRegistry::default_impl(const AttentionOpContext& ctx) const {
    for (auto& i : impls_)
        if (i->supports(ctx)) return i.get();
    throw ConfigurationError("no attention implementation supports this configuration");
}

// ---------------------------------------------------------------------------------
// Norm
// ---------------------------------------------------------------------------------
namespace {
void hip_rms_norm(const RMSNormOpContext& c, const Tensor& in, const Tensor& w, Tensor& out, hipStream_t s) {
    efm_check(efm_rms_norm(c.batch_size, c.hidden_size, c.eps, in.data_ptr(), w.data_ptr(), out.data_ptr(), s),
              "rms_norm");
}
void hip_fused_add_rms_norm(const RMSNormOpContext& c, Tensor& inout, Tensor& residual, const Tensor& w,
                            hipStream_t s) {
    efm_check(efm_fused_add_rms_norm(c.batch_size, c.hidden_size, c.eps, inout.data_ptr(), residual.data_ptr(),
                                     w.data_ptr(), s),
              "fused_add_rms_norm");
}
class HipNormOp final : public NormOp {
public:
    std::string impl_id() const override { return "hip_gfx950_norm"; }
    bool supports(const RMSNormOpContext& c) const override {
        return c.dtype == DType::BFloat16 && c.hidden_size % 8 == 0 && c.hidden_size <= 16384;
    }
    RMSNormForwardFn rms_norm_forward_fn() const override { return &hip_rms_norm; }
    FusedAddRMSNormForwardFn fused_add_rms_norm_forward_fn() const override { return &hip_fused_add_rms_norm; }
};
}  // namespace

NormOpRegistry::NormOpRegistry() { impls_.push_back(std::make_unique<HipNormOp>()); }
NormOpRegistry& NormOpRegistry::instance() {
    static NormOpRegistry r;
    return r;
}
NormOp* NormOpRegistry::find_impl_by_id(const std::string& id) const {
    for (auto& i : impls_)
        if (i->impl_id() == id) return i.get();
    return nullptr;
}
NormOp* NormOpRegistry::default_impl(const RMSNormOpContext& ctx) const {
    for (auto& i : impls_)
        if (i->supports(ctx)) return i.get();
    throw ConfigurationError("no norm implementation supports this configuration");
}

// ---------------------------------------------------------------------------------
// Activation
// ---------------------------------------------------------------------------------
namespace {
class HipActivationOp final : public ActivationOp {
public:
    std::string impl_id() const override { return "hip_gfx950_silu_and_mul"; }
    bool supports(const ActivationOpContext& c) const override {
        return c.dtype == DType::BFloat16 && c.kind == ActivationKind::kSilu && c.hidden_size % 8 == 0;
    }
    void act_and_mul(const ActivationOpContext& c, const Tensor& in, Tensor& out, hipStream_t s) override {
        if (c.kind != ActivationKind::kSilu) throw ConfigurationError("activation operator only supports silu");
        efm_check(efm_act_and_mul(c.batch_size, c.hidden_size,
                                  c.input_layout == ActivationInputLayout::kUpGate ? EFM_LAYOUT_UP_GATE
                                                                                   : EFM_LAYOUT_GATE_UP,
                                  in.data_ptr(), out.data_ptr(), s),
                  "act_and_mul");
    }
};
}  // namespace

ActivationOpRegistry::ActivationOpRegistry() { impls_.push_back(std::make_unique<HipActivationOp>()); }
ActivationOpRegistry& ActivationOpRegistry::instance() {
    static ActivationOpRegistry r;
    return r;
}
ActivationOp* ActivationOpRegistry::find_impl_by_id(const std::string& id) const {
    for (auto& i : impls_)
        if (i->impl_id() == id) return i.get();
    return nullptr;
}
ActivationOp* ActivationOpRegistry::default_impl(const ActivationOpContext& ctx) const {
    for (auto& i : impls_)
        if (i->supports(ctx)) return i.get();
    throw ConfigurationError("no activation implementation supports this configuration");
}

// ---------------------------------------------------------------------------------
// Linear
// ---------------------------------------------------------------------------------
std::string linear_shape_sig(const LinearShape& s) {
    return "m=" + std::to_string(s.m) + "|input=" + std::to_string((int)s.input) +
           "|weight=" + std::to_string((int)s.weight) + "|output=" + std::to_string((int)s.output) +
           "|in_features=" + std::to_string(s.in_features) + "|out_features=" + std::to_string(s.out_features);
}

namespace {
// Grow-only per-device scratch for the split-K prefill GEMMs (the reference's linear impls
// take theirs from StaticBufferManager::get_cache_buf, src/utils/memory.h:31-109). Grows
// only outside graph capture: decode (m = 1) never needs it.
void* linear_scratch(size_t bytes, int32_t device_id, size_t* have) {
    static std::mutex mu;
    static std::map<int32_t, Tensor> bufs;
    std::lock_guard<std::mutex> lock(mu);
    Tensor& t = bufs[device_id];
    if (t.empty() || t.nbytes() < bytes) t = Tensor::empty({(int64_t)bytes}, DType::UInt8, Device::GPU, device_id);
    *have = t.nbytes();
    return t.data_ptr();
}

class HipLinearImpl final : public LinearImpl {
public:
    std::string impl_id() const override { return "hip_gfx950_linear"; }
    bool supports(const LinearOpContext& c) const override {
        const auto& s = c.shape;
        if (s.input != DType::BFloat16 || s.weight != DType::BFloat16) return false;
        if (s.output != DType::BFloat16 && s.output != DType::Float32) return false;
        return s.in_features % (s.m == 1 ? 8 : 32) == 0;
    }
    void forward(const LinearOpContext& c, const Tensor& w, const Tensor* bias, const Tensor& in, Tensor& out,
                 hipStream_t s) override {
        // The shape's own figure, not the scratch's capacity: the kernels chosen must not
        // depend on how far earlier, longer prompts have grown the buffer.
        const size_t need = efm_linear_workspace_bytes(c.shape.m, c.shape.in_features, c.shape.out_features);
        size_t have = 0;
        void* ws = need > 0 ? linear_scratch(need, w.device().second, &have) : nullptr;
        efm_check(efm_linear_ws(c.shape.m, c.shape.in_features, c.shape.out_features, in.data_ptr(), w.data_ptr(),
                                bias ? bias->data_ptr() : nullptr, out.data_ptr(),
                                c.shape.output == DType::Float32 ? EFM_DTYPE_F32 : EFM_DTYPE_BF16, ws, need, s),
                  "linear " + c.layer_prefix);
    }
};
}  // namespace

LinearOpRegistry::LinearOpRegistry() { impls_.push_back(std::make_unique<HipLinearImpl>()); }
LinearOpRegistry& LinearOpRegistry::instance() {
    static LinearOpRegistry r;
    return r;
}
LinearImpl* LinearOpRegistry::find_impl_by_id(const std::string& id) const {
    for (auto& i : impls_)
        if (i->impl_id() == id) return i.get();
    return nullptr;
}
LinearImpl* LinearOpRegistry::default_impl(const LinearOpContext& ctx) const {
    for (auto& i : impls_)
        if (i->supports(ctx)) return i.get();
    throw ConfigurationError("no linear implementation supports " + linear_shape_sig(ctx.shape));
}

// ---------------------------------------------------------------------------------
// Fused gate/up + SwiGLU
// ---------------------------------------------------------------------------------
namespace {
class HipSwigluOp final : public FusedGateUpActivationOp {
public:
    std::string impl_id() const override { return "hip_gfx950_swiglu"; }
    bool supports(const FusedGateUpActivationContext& c) const override {
        return c.dtype == DType::BFloat16 && c.hidden % (c.m == 1 ? 8 : 32) == 0;
    }
    FusedGateUpActivationState prepare(const FusedGateUpActivationContext& c, const Tensor& w) override {
        FusedGateUpActivationState st;
        if (!supports(c)) {
            st.unavailable_reason = "unsupported shape or dtype";
        } else if (w.shape().size() != 2 || w.shape()[0] != 2 * c.intermediate || w.shape()[1] != c.hidden) {
            st.unavailable_reason = "weight is not the fused [up; gate] matrix";
        } else {
            st.available = true;
        }
        return st;
    }
    bool run(const FusedGateUpActivationContext& c, const Tensor& w, const Tensor& in, Tensor& out,
             hipStream_t s) override {
        if (!supports(c)) return false;  // fast path unavailable -> caller falls back
        const size_t need = efm_fused_gate_up_swiglu_workspace_bytes(c.m, c.hidden, c.intermediate);
        size_t have = 0;
        void* ws = need > 0 ? linear_scratch(need, w.device().second, &have) : nullptr;
        efm_check(efm_fused_gate_up_swiglu_ws(c.m, c.hidden, c.intermediate, in.data_ptr(), w.data_ptr(),
                                              out.data_ptr(), ws, need, s),
                  "fused_gate_up_swiglu");
        return true;
    }
};
}  // namespace

FusedGateUpActivationRegistry::FusedGateUpActivationRegistry() {
    impls_.push_back(std::make_unique<HipSwigluOp>());
}
FusedGateUpActivationRegistry& FusedGateUpActivationRegistry::instance() {
    static FusedGateUpActivationRegistry r;
    return r;
}
FusedGateUpActivationOp* FusedGateUpActivationRegistry::find_impl_by_id(const std::string& id) const {
    for (auto& i : impls_)
        if (i->impl_id() == id) return i.get();
    return nullptr;
}
FusedGateUpActivationOp* FusedGateUpActivationRegistry::default_impl(const FusedGateUpActivationContext& c) const {
    for (auto& i : impls_)
        if (i->supports(c)) return i.get();
    return nullptr;
}

}  // namespace edge_fm
