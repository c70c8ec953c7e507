#include "operators.hpp"

#include "engine.hpp"

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

// The records used when the engine config names no table file (the role of the
// reference's engine_default table): each op kind resolves to this library's impls, and at
// stage "decode" the attention of a layer is the split attention whose partials merge in
// the o_proj prologue (impls that do not support a shape fall back to the registry
// default, attention.cu:257-273). The one-launch norm + QKV + attention impl is selected
// by a table record: on MI355X its in-kernel hand-off of the query across XCDs costs
// more than the kernel boundary it saves.
static std::vector<OperatorImplRecord> builtin_records() {
    std::vector<OperatorImplRecord> out;
    const char* recs[][4] = {{"linear", "", "", "hip_gfx950_linear"},
                             {"linear", "attention_output", "decode", "hip_gfx950_decode_merge_o_proj"},
                             {"attention", "", "", "hip_gfx950_attention"},
                             {"attention", "", "decode", "hip_gfx950_decode_split_attention"},
                             {"norm", "", "", "hip_gfx950_norm"},
                             {"activation", "", "", "hip_gfx950_silu_and_mul"},
                             {"fused_gate_up_activation", "", "", "hip_gfx950_swiglu"}};
    for (const char* model : {"qwen2_5", "qwen2_5_vl"}) {
        for (auto& k : recs) {
            OperatorImplRecord r;
            r.model_name = model;
            r.hw_profile = "rocm";
            r.op_kind = k[0];
            r.layer_role = k[1];
            r.stage = k[2];
            r.impl_id = k[3];
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
    // A table file replaces the built-in records (the reference reads one table file);
    // queries it has no record for resolve to the registry defaults.
    std::vector<OperatorImplRecord> recs;
    if (path.empty()) recs = builtin_records();
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
std::string attention_shape_sig(uint32_t num_qo_heads, uint32_t num_kv_heads, uint32_t head_dim) {
    return "num_qo_heads=" + std::to_string(num_qo_heads) + "|num_kv_heads=" + std::to_string(num_kv_heads) +
           "|head_dim=" + std::to_string(head_dim);
}

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

class HipAttentionOp : public AttentionOp {
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

// Decode-stage attention impls. Both compute the same attention as HipAttentionOp (its
// forward_prefill / forward_decode run for direct calls); what they add is how a decode
// layer is launched, which the engine reads from the impl id:
//   hip_gfx950_decode_fused_qkv_attention  the input norm + QKV + split attention in one
//       launch (efm_decode_norm_qkv_attention), partials merged in the o_proj prologue
//   hip_gfx950_decode_split_attention      norm + QKV, then the split attention, partials
//       merged in the o_proj prologue
// Both need the merge to fold into o_proj (efm_decode_attention_merge_o_proj_supported:
// up to 24 splits for query widths up to 1024, 12 up to 2048); the fused launch also a
// text model (rotate-on-read cache), head_dim 128 and
// efm_decode_norm_qkv_attention_supported (128-key splits).
class HipDecodeSplitAttentionOp : public HipAttentionOp {
public:
    std::string impl_id() const override { return "hip_gfx950_decode_split_attention"; }
    bool supports(const AttentionOpContext& c) const override {
        if (!HipAttentionOp::supports(c) || c.decode_max_kv_len == 0) return false;
        const efm_attention_ctx cc = to_c_ctx(c);
        return efm_decode_attention_merge_o_proj_supported(&cc, c.decode_max_kv_len) == EFM_OK;
    }
};

class HipDecodeFusedQkvAttentionOp final : public HipDecodeSplitAttentionOp {
public:
    std::string impl_id() const override { return "hip_gfx950_decode_fused_qkv_attention"; }
    bool supports(const AttentionOpContext& c) const override {
        if (!HipDecodeSplitAttentionOp::supports(c) || c.decode_hidden == 0) return false;
        if (c.pos_encoding != AttentionPosEncoding::kRoPELlama) return false;
        efm_attention_ctx cc = to_c_ctx(c);
        cc.k_already_prerotated = EFM_K_PREROTATED_EXCEPT_NEWEST;
        return efm_decode_norm_qkv_attention_supported(&cc, (int32_t)c.decode_hidden, c.decode_max_kv_len) == EFM_OK;
    }
};

}  // namespace

// default preference: split partials, fused launch, generic attention
AttentionOpRegistry::AttentionOpRegistry() {
    impls_.push_back(std::make_unique<HipDecodeSplitAttentionOp>());
    impls_.push_back(std::make_unique<HipDecodeFusedQkvAttentionOp>());
    impls_.push_back(std::make_unique<HipAttentionOp>());
}
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
std::string infer_layer_role(const std::string& p) {
    if (p.find("lm_head") != std::string::npos) return "lm_head";
    if (p.find("qkv_fused") != std::string::npos) return "fused_qkv";
    if (p.find("gate_up_fused") != std::string::npos) return "fused_gate_up";
    if (p.find(".o_proj") != std::string::npos) return "attention_output";
    if (p.find(".down_proj") != std::string::npos) return "mlp_down";
    return "linear";
}

std::string stage_key(ModelStage stage) { return stage == ModelStage::Decode ? "decode" : "prefill"; }

std::string LinearLayer::LinearShapeSignature::to_string() const {
    return "m=" + std::to_string(m) + "|input=" + std::to_string((int)input_dtype) +
           "|weight=" + std::to_string((int)weight_dtype) + "|output=" + std::to_string((int)output_dtype) +
           "|in_features=" + std::to_string(in_features) + "|out_features=" + std::to_string(out_features);
}

namespace {

bool plain_bf16(const LinearLayer::LinearOpContext& c, const LinearLayer::WeightSet& ws) {
    const auto& s = c.shape;
    if (ws.quant_type_ != LinearLayer::QuantType::FP16_BF16 || ws.weight_ == nullptr) return false;
    if (s.input_dtype != DType::BFloat16 || s.weight_dtype != DType::BFloat16) return false;
    if (s.output_dtype != DType::BFloat16 && s.output_dtype != DType::Float32) return false;
    return s.m >= 1 && s.in_features % (s.m == 1 ? 8u : 32u) == 0;
}

}  // namespace

// One grow-only split-K scratch per device, shared by every prefill projection (linear
// impls, the prefill source ops, the fused gate/up op), in the role of the reference's
// StaticBufferManager::get_cache_buf (src/utils/memory.h:31-109): all of them run in
// stream order, so one buffer sized to the largest need serves every prompt length. It
// only grows: the device is synchronised first, so no launch still reads the old one.
// Decode GEMVs (m = 1) need none, so captured decode graphs never hold it.
namespace {
struct SharedLinearScratch {
    std::mutex mu;
    std::map<int32_t, Tensor> bufs;
    std::map<int32_t, uint64_t> generation;   // bumped whenever a device's buffer is replaced
} g_linear_scratch;
}  // namespace

void* linear_scratch(size_t bytes, int32_t device_id, size_t* have) {
    std::lock_guard<std::mutex> lock(g_linear_scratch.mu);
    Tensor& t = g_linear_scratch.bufs[device_id];
    if (bytes > 0 && (t.empty() || t.nbytes() < bytes)) {
        if (!t.empty()) hip_check(hipDeviceSynchronize(), "linear scratch grow");
        t = Tensor();
        t = Tensor::empty({(int64_t)bytes}, DType::UInt8, Device::GPU, device_id);
        ++g_linear_scratch.generation[device_id];
    }
    *have = t.empty() ? 0 : t.nbytes();
    return t.empty() ? nullptr : t.data_ptr();
}

uint64_t linear_scratch_generation(int32_t device_id) {
    std::lock_guard<std::mutex> lock(g_linear_scratch.mu);
    return g_linear_scratch.generation[device_id];
}

size_t linear_scratch_bytes(int32_t device_id) {
    std::lock_guard<std::mutex> lock(g_linear_scratch.mu);
    auto it = g_linear_scratch.bufs.find(device_id);
    return (it == g_linear_scratch.bufs.end() || it->second.empty()) ? 0 : it->second.nbytes();
}

namespace {
// This library's GEMV (m = 1) / MFMA GEMM (m > 1). prepare() records the split-K scratch
// the kernel plan for this shape uses (zero for most shapes, and always for m = 1);
// forward() takes it from the shared device scratch, which only grows when a new shape
// needs more (never at m = 1, so a decode step can be captured into a graph).
class HipLinearImpl : public LinearLayer::LinearImpl {
public:
    std::string impl_id() const override { return "hip_gfx950_linear"; }
    bool supports(const LinearLayer::LinearOpContext& c, const LinearLayer::WeightSet& ws) const override {
        return plain_bf16(c, ws);
    }
    void prepare(LinearLayer&, const LinearLayer::LinearOpContext& c, const LinearLayer::WeightSet& ws,
                 const Tensor&, Tensor&, hipStream_t, LinearLayer::CachedDescriptors& cached) override {
        if (cached.prepared_) return;
        cached.workspace_bytes_ = efm_linear_workspace_bytes(c.shape.m, c.shape.in_features, c.shape.out_features);
        cached.prepared_ = true;
    }
    void forward(LinearLayer& owner, const LinearLayer::LinearOpContext& c, const LinearLayer::WeightSet& ws,
                 const Tensor& in, Tensor& out, hipStream_t s, LinearLayer::CachedDescriptors& cached) override {
        prepare(owner, c, ws, in, out, s, cached);
        size_t have = 0;
        void* scratch = cached.workspace_bytes_ > 0
                            ? linear_scratch(cached.workspace_bytes_, ws.weight_->device().second, &have)
                            : nullptr;
        efm_check(efm_linear_ws(c.shape.m, c.shape.in_features, c.shape.out_features, in.data_ptr(),
                                ws.weight_->data_ptr(), ws.bias_ ? ws.bias_->data_ptr() : nullptr, out.data_ptr(),
                                c.shape.output_dtype == DType::Float32 ? EFM_DTYPE_F32 : EFM_DTYPE_BF16, scratch,
                                have, s),
                  "linear " + c.layer_prefix);
    }
};

// The o_proj of a decode layer whose attention left split partials: the engine runs the
// merge in this GEMV's prologue (efm_decode_attention_merge_o_proj). Called as a plain
// linear (a merged attention output in), it is the GEMV.
class HipDecodeMergeOProjImpl final : public HipLinearImpl {
public:
    std::string impl_id() const override { return "hip_gfx950_decode_merge_o_proj"; }
    bool supports(const LinearLayer::LinearOpContext& c, const LinearLayer::WeightSet& ws) const override {
        return c.stage == ModelStage::Decode && c.layer_role == "attention_output" && c.shape.m == 1 &&
               c.shape.output_dtype == DType::BFloat16 && ws.bias_ == nullptr && plain_bf16(c, ws);
    }
};

// Prefill projections through PrefillLinearSourceOp::try_forward, the layered GEMM when
// it declines (the reference's cutlass_prefill_linear_source_op, linear_impl.cu:708-770).
class HipPrefillSourceOpLinearImpl final : public LinearLayer::LinearImpl {
public:
    std::string impl_id() const override { return "hip_gfx950_prefill_linear_source_op"; }
    bool supports(const LinearLayer::LinearOpContext& c, const LinearLayer::WeightSet& ws) const override {
        return c.stage == ModelStage::Prefill && (c.layer_role == "fused_qkv" || c.layer_role == "attention_output") &&
               c.shape.output_dtype == DType::BFloat16 && plain_bf16(c, ws);
    }
    void prepare(LinearLayer&, const LinearLayer::LinearOpContext&, const LinearLayer::WeightSet&, const Tensor&,
                 Tensor&, hipStream_t, LinearLayer::CachedDescriptors& cached) override {
        cached.selected_impl_id_ = impl_id();
    }
    void forward(LinearLayer& owner, const LinearLayer::LinearOpContext& c, const LinearLayer::WeightSet& ws,
                 const Tensor& in, Tensor& out, hipStream_t s, LinearLayer::CachedDescriptors& cached) override {
        prepare(owner, c, ws, in, out, s, cached);
        PrefillLinearSourceOp* op = owner.prefill_linear_source_op();
        if (op != nullptr && op->try_forward(c.layer_role, 0, in, *ws.weight_, ws.bias_, out, s)) return;
        LinearLayer::LinearImpl* fallback = LinearOpRegistry::instance().find_impl_by_id("hip_gfx950_linear");
        check<InternalError>(fallback != nullptr, "LinearLayer: hip_gfx950_linear fallback impl is missing");
        fallback->forward(owner, c, ws, in, out, s, cached);
    }
};

// A shape-only weight descriptor (no storage) so that impls can be resolved and planned
// before weights are loaded; supports() reads only dtypes and shapes.
Tensor shape_only(std::vector<int64_t> shape, int32_t device_id) {
    return Tensor::view(nullptr, std::move(shape), DType::BFloat16, Device::GPU, device_id);
}

}  // namespace

LinearOpRegistry::LinearOpRegistry() {
    impls_.push_back(std::make_unique<HipDecodeMergeOProjImpl>());
    impls_.push_back(std::make_unique<HipLinearImpl>());
    impls_.push_back(std::make_unique<HipPrefillSourceOpLinearImpl>());
}
LinearOpRegistry& LinearOpRegistry::instance() {
    static LinearOpRegistry r;
    return r;
}
LinearLayer::LinearImpl* LinearOpRegistry::find_impl_by_id(const std::string& id) const {
    for (auto& i : impls_)
        if (i->impl_id() == id) return i.get();
    return nullptr;
}
LinearLayer::LinearImpl* LinearOpRegistry::default_impl(const LinearLayer::LinearOpContext& ctx,
                                                        const LinearLayer::WeightSet& ws) const {
    for (auto& i : impls_)
        if (i->supports(ctx, ws)) return i.get();
    return nullptr;
}

LinearLayer::LinearLayer(const std::string& layer_prefix, const EngineConfig& engine_config, uint32_t in_features,
                         uint32_t out_features, std::string layer_name)
    : LinearLayer(layer_prefix, infer_layer_role(layer_prefix), engine_config, in_features, out_features,
                  std::move(layer_name)) {}

LinearLayer::LinearLayer(const std::string& layer_prefix, std::string layer_role, const EngineConfig& engine_config,
                         uint32_t in_features, uint32_t out_features, std::string layer_name)
    : prefix_(layer_prefix), role_(std::move(layer_role)), name_(std::move(layer_name)),
      model_name_(engine_config.model_name()), hw_profile_(engine_config.hw_profile()),
      table_path_(engine_config.operator_table_path()), in_(in_features), out_(out_features),
      source_op_(std::make_unique<PrefillLinearSourceOp>(engine_config)) {
    weight_ = shape_only({(int64_t)out_, (int64_t)in_}, engine_config.device_id());
    ws_.weight_ = &weight_;
}

LinearLayer::~LinearLayer() = default;

void LinearLayer::load_weights(const Tensor& weight, const Tensor* bias) {
    check<ModelNotLoadedError>(weight.shape().size() == 2 && weight.shape()[0] == out_ && weight.shape()[1] == in_,
                               "LinearLayer " + prefix_ + ": weight must be [" + std::to_string(out_) + ", " +
                                   std::to_string(in_) + "]");
    check<ModelNotLoadedError>(weight.dtype() == DType::BFloat16, "LinearLayer " + prefix_ + ": weight must be bf16");
    weight_ = weight;
    ws_.weight_ = &weight_;
    if (bias != nullptr) {
        check<ModelNotLoadedError>(bias->numel() == out_ && bias->dtype() == DType::BFloat16,
                                   "LinearLayer " + prefix_ + ": bias must be bf16 [" + std::to_string(out_) + "]");
        bias_ = *bias;
        ws_.bias_ = &bias_;
    } else {
        bias_ = Tensor();
        ws_.bias_ = nullptr;
    }
    reset_operator_impl_cache();
}

const Tensor* LinearLayer::weight_tensor(ModelStage) const { return weight_.empty() ? nullptr : &weight_; }
const Tensor* LinearLayer::bias_tensor(ModelStage) const { return bias_.empty() ? nullptr : &bias_; }

void LinearLayer::reset_operator_impl_cache() {
    cache_.clear();
    if (source_op_) source_op_->reset_runtime_caches();
}

LinearLayer::LinearOpContext LinearLayer::make_ctx(int32_t m, DType input_dtype, DType output_dtype,
                                                   ModelStage stage) const {
    LinearOpContext c;
    c.layer_prefix = prefix_;
    c.layer_role = role_;
    c.stage = stage;
    c.shape.m = m;
    c.shape.input_dtype = input_dtype;
    c.shape.weight_dtype = weight_.dtype();
    c.shape.output_dtype = output_dtype;
    c.shape.in_features = in_;
    c.shape.out_features = out_;
    c.has_bias = ws_.bias_ != nullptr;
    return c;
}

LinearLayer::CachedDescriptors& LinearLayer::cache_slot(ModelStage stage, int32_t m, DType output_dtype) {
    return cache_[std::make_tuple((int)stage, m, (int)output_dtype)];
}

LinearLayer::LinearImpl* LinearLayer::resolve_impl(const LinearOpContext& ctx, const WeightSet& ws,
                                                   CachedDescriptors& cached) const {
    if (!cached.selected_impl_id_.empty()) {
        if (LinearImpl* impl = LinearOpRegistry::instance().find_impl_by_id(cached.selected_impl_id_)) return impl;
        cached.selected_impl_id_.clear();
    }
    OperatorQuery q;
    q.op_kind = "linear";
    q.layer_role = ctx.layer_role;
    q.op_name = ctx.layer_prefix;
    q.stage = stage_key(ctx.stage);
    q.shape_sig = ctx.shape.to_string();
    if (auto rec = OperatorImplTable::instance().resolve(model_name_, hw_profile_, table_path_, q)) {
        LinearImpl* impl = LinearOpRegistry::instance().find_impl_by_id(rec->impl_id);
        if (impl == nullptr)
            throw ConfigurationError("LinearLayer: operator_impl_table selected unknown impl '" + rec->impl_id +
                                     "' for layer '" + prefix_ + "'");
        if (!impl->supports(ctx, ws))
            throw ConfigurationError("LinearLayer: operator_impl_table selected unsupported impl '" + rec->impl_id +
                                     "' for layer '" + prefix_ + "' (" + stage_key(ctx.stage) + ", " +
                                     ctx.shape.to_string() + ")");
        cached.selected_impl_id_ = impl->impl_id();
        cached.selected_impl_params_ = rec->impl_params;
        return impl;
    }
    if (LinearImpl* impl = LinearOpRegistry::instance().default_impl(ctx, ws)) {
        cached.selected_impl_id_ = impl->impl_id();
        cached.selected_impl_params_ = Json::object();
        return impl;
    }
    throw ConfigurationError("LinearLayer: no supported implementation found for layer '" + prefix_ + "' (" +
                             ctx.shape.to_string() + ")");
}

std::string LinearLayer::selected_impl_id(ModelStage stage, int32_t m, DType output_dtype) {
    const LinearOpContext ctx = make_ctx(m, DType::BFloat16, output_dtype, stage);
    return resolve_impl(ctx, ws_, cache_slot(stage, m, output_dtype))->impl_id();
}

void LinearLayer::forward_fp16_bf16(const Tensor& input, Tensor& output, hipStream_t stream, ModelStage stage) {
    check<InvalidRequestError>(!weight_.empty(), "LinearLayer " + prefix_ + ": weights are not loaded");
    check<InvalidRequestError>(input.shape().size() == 2 && input.shape()[1] == in_,
                               "LinearLayer " + prefix_ + ": input must be [m, " + std::to_string(in_) + "]");
    const int32_t m = (int32_t)input.shape()[0];
    check<InvalidRequestError>(output.numel() == (int64_t)m * out_,
                               "LinearLayer " + prefix_ + ": output must hold [m, " + std::to_string(out_) + "]");
    const LinearOpContext ctx = make_ctx(m, input.dtype(), output.dtype(), stage);
    CachedDescriptors& cached = cache_slot(stage, m, output.dtype());
    LinearImpl* impl = resolve_impl(ctx, ws_, cached);
    impl->forward(*this, ctx, ws_, input, output, stream, cached);
}

// ---------------------------------------------------------------------------------
// Prefill source ops
// ---------------------------------------------------------------------------------
namespace {
bool bf16_matrix(const Tensor& t, int64_t rows, int64_t cols) {
    return t.dtype() == DType::BFloat16 && t.shape().size() == 2 && (rows < 0 || t.shape()[0] == rows) &&
           (cols < 0 || t.shape()[1] == cols) && !t.empty();
}
}  // namespace

PrefillLinearSourceOp::PrefillLinearSourceOp(const EngineConfig& config) : device_id_(config.device_id()) {}
PrefillLinearSourceOp::~PrefillLinearSourceOp() = default;
void PrefillLinearSourceOp::reset_runtime_caches() {}

bool PrefillLinearSourceOp::try_forward(const std::string& role, int32_t, const Tensor& input, const Tensor& weight,
                                        const Tensor* bias, Tensor& output, hipStream_t stream) {
    if (role != "fused_qkv" && role != "attention_output" && role != "mlp_down" && role != "linear") return false;
    if (!bf16_matrix(input, -1, -1) || !bf16_matrix(weight, -1, input.shape()[1])) return false;
    const int64_t m = input.shape()[0], k = input.shape()[1], n = weight.shape()[0];
    if (m < 2 || k % 32 != 0 || output.dtype() != DType::BFloat16 || output.numel() != m * n) return false;
    if (bias != nullptr && (bias->dtype() != DType::BFloat16 || bias->numel() != n)) return false;
    const size_t need = efm_linear_workspace_bytes(m, k, n);
    size_t have = 0;
    void* ws = need > 0 ? linear_scratch(need, device_id_, &have) : nullptr;
    efm_check(efm_linear_ws(m, k, n, input.data_ptr(), weight.data_ptr(), bias ? bias->data_ptr() : nullptr,
                            output.data_ptr(), EFM_DTYPE_BF16, ws, have, stream),
              "prefill linear source op (" + role + ")");
    return true;
}

PrefillMlpSourceOp::PrefillMlpSourceOp(const EngineConfig& config) : device_id_(config.device_id()) {}
PrefillMlpSourceOp::~PrefillMlpSourceOp() = default;
void PrefillMlpSourceOp::reset_runtime_caches() {
    intermediate_ = Tensor();
    ++generation_;
}

bool PrefillMlpSourceOp::try_forward(int32_t, const Tensor& input, const Tensor& gate_up_weight,
                                     const Tensor& down_weight, Tensor& output, hipStream_t stream) {
    if (!bf16_matrix(input, -1, -1)) return false;
    const int64_t m = input.shape()[0], h = input.shape()[1];
    if (m < 2 || h % 32 != 0 || !bf16_matrix(gate_up_weight, -1, h) || gate_up_weight.shape()[0] % 2 != 0)
        return false;
    const int64_t inter = gate_up_weight.shape()[0] / 2;
    if (inter % 32 != 0 || !bf16_matrix(down_weight, h, inter)) return false;
    if (output.dtype() != DType::BFloat16 || output.numel() != m * h) return false;
    if (intermediate_.empty() || intermediate_.numel() < m * inter) {
        if (!intermediate_.empty()) hip_check(hipDeviceSynchronize(), "prefill mlp intermediate grow");
        intermediate_ = Tensor();
        intermediate_ = Tensor::empty({m, inter}, DType::BFloat16, Device::GPU, device_id_);
        ++generation_;
    }
    // both launches share the scratch (stream order): grown once, to the larger need
    const size_t need_gu = efm_fused_gate_up_swiglu_workspace_bytes(m, h, inter);
    const size_t need_d = efm_linear_workspace_bytes(m, inter, h);
    size_t have = 0;
    void* ws = (need_gu | need_d) ? linear_scratch(std::max(need_gu, need_d), device_id_, &have) : nullptr;
    efm_check(efm_fused_gate_up_swiglu_ws(m, h, inter, input.data_ptr(), gate_up_weight.data_ptr(),
                                          intermediate_.data_ptr(), need_gu ? ws : nullptr, need_gu ? have : 0,
                                          stream),
              "prefill mlp source op (gate/up + SwiGLU)");
    efm_check(efm_linear_ws(m, inter, h, intermediate_.data_ptr(), down_weight.data_ptr(), nullptr, output.data_ptr(),
                            EFM_DTYPE_BF16, need_d ? ws : nullptr, need_d ? have : 0, stream),
              "prefill mlp source op (down)");
    return true;
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
