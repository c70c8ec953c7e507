#include "layers.hpp"

#include <climits>
#include <map>
#include <mutex>
#include <numeric>

namespace edge_fm {

namespace {

std::string stage_str(ModelStage s) { return s == ModelStage::Decode ? "decode" : "prefill"; }
size_t slot_of(ModelStage s) { return s == ModelStage::Decode ? 1u : 0u; }

void check_device(const Tensor& t, int32_t device_id, const std::string& name) {
    const auto [dev, id] = t.device();
    check<DeviceError>(dev == Device::GPU && id == device_id, name + " tensor must be on the same device as the layer");
    check<InvalidRequestError>(!t.empty(), name + " tensor is empty");
}

// Named device buffers that only grow, zero-filled when (re)allocated, one per (name,
// device): the layers' workspaces (the role of StaticBufferManager::get_cache_buf,
// src/utils/device/memory.h:18-113). A buffer is replaced only after the device is idle.
Tensor cache_buf(const std::string& name, size_t bytes, int32_t device_id) {
    static std::mutex mu;
    static std::map<std::pair<std::string, int32_t>, Tensor> bufs;
    std::lock_guard<std::mutex> lock(mu);
    Tensor& t = bufs[{name, device_id}];
    if (t.empty() || t.nbytes() < bytes) {
        if (!t.empty()) hip_check(hipDeviceSynchronize(), "workspace grow");
        t = Tensor::zeros({(int64_t)std::max<size_t>(bytes, 256)}, DType::UInt8, Device::GPU, device_id);
    }
    return t;
}

uint32_t cfg_u32(const Json& j, const char* key, uint32_t def) { return (uint32_t)j.get_int(key, (int64_t)def); }

// The impl id the operator table selects for q, after the reference layers' rule
// (attention.cu:211-276, layernorm.cu:97-150, activation.cu:61-105): no record -> the
// registry default; a record naming an unknown impl -> ConfigurationError.
template <class Registry, class Op>
Op* table_impl(const std::string& model, const std::string& hw, const std::string& table, const OperatorQuery& q,
               const char* layer, Json* params) {
    auto rec = OperatorImplTable::instance().resolve(model, hw, table, q);
    if (!rec) return nullptr;
    Op* op = Registry::instance().find_impl_by_id(rec->impl_id);
    if (op == nullptr)
        throw ConfigurationError(std::string(layer) + ": operator_impl_table selected unknown impl '" + rec->impl_id +
                                 "'");
    if (params) *params = rec->impl_params;
    return op;
}

}  // namespace

const std::unordered_map<std::string, Tensor>& layer_stage_weights(const EngineConfig& cfg,
                                                                   const std::vector<std::string>& any_of) {
    WeightLoader& loader = WeightLoader::instance();
    if (loader.has_stage(ModelStage::Prefill)) {
        const auto& have = loader.get(ModelStage::Prefill);
        for (const auto& n : any_of)
            if (have.count(n)) return have;
    }
    loader.load_weights_from_file(cfg.prefill_model_path(), ModelStage::Prefill, cfg.device_id(),
                                  cfg.model_name() == "qwen2_5_vl");
    return loader.get(ModelStage::Prefill);
}

// =================================================================================
// AttentionLayer
// =================================================================================
AttentionLayer::AttentionLayer(const EngineConfig& cfg, std::string layer_name)
    : model_name_(cfg.model_name()), hw_profile_(cfg.hw_profile()), table_path_(cfg.operator_table_path()),
      layer_name_(std::move(layer_name)), device_id_(cfg.device_id()) {
    const Json& m = cfg.model_config();
    const std::string dt = m.get_string("torch_dtype", "float16");
    dtype_ = dtype_from_string(dt);
    check<ConfigurationError>(dtype_ == DType::Float16 || dtype_ == DType::BFloat16,
                              "AttentionLayer only supports Float16 or BFloat16, got torch_dtype=" + dt);
    num_qo_heads_ = cfg_u32(m, "num_attention_heads", 32);
    num_kv_heads_ = cfg_u32(m, "num_key_value_heads", num_qo_heads_);
    const uint32_t hidden = cfg_u32(m, "hidden_size", 4096);
    check<ConfigurationError>(num_qo_heads_ > 0 && hidden % num_qo_heads_ == 0,
                              "hidden_size must be divisible by num_attention_heads. Got hidden_size=" +
                                  std::to_string(hidden) + ", num_attention_heads=" + std::to_string(num_qo_heads_));
    head_dim_ = hidden / num_qo_heads_;
    rope_theta_ = (float)m.get_double("rope_theta", 1000000.0);
    if (m.contains("rope_scaling") && m.at("rope_scaling").is_object()) {
        const Json& rs = m.at("rope_scaling");
        if (rs.contains("factor")) rope_scale_ = (float)rs.get_double("factor", 1.0);
        std::string type = rs.get_string("type");
        if (type.empty()) type = rs.get_string("rope_type");
        if (type == "mrope") rope_mode_ = RoPEMode::kMRoPE;
    }
}

AttentionOpContext AttentionLayer::base_ctx() const {
    AttentionOpContext c;
    c.num_qo_heads = num_qo_heads_;
    c.num_kv_heads = num_kv_heads_;
    c.head_dim = head_dim_;
    c.rope_theta = rope_theta_;
    c.rope_scale = rope_scale_;
    c.dtype = dtype_;
    c.pos_encoding = rope_mode_ == RoPEMode::kRoPELlama ? AttentionPosEncoding::kRoPELlama : AttentionPosEncoding::kNone;
    c.device_id = device_id_;
    return c;
}

AttentionOp* AttentionLayer::resolve_impl(ModelStage stage) const {
    const size_t s = slot_of(stage);
    if (selected_[s]) return selected_[s];
    AttentionOpContext ctx = base_ctx();
    OperatorQuery q;
    q.op_kind = "attention";
    q.op_name = "attention";
    q.stage = stage_str(stage);
    q.shape_sig = attention_shape_sig(num_qo_heads_, num_kv_heads_, head_dim_);
    Json params = Json::object();
    AttentionOp* op = table_impl<AttentionOpRegistry, AttentionOp>(model_name_, hw_profile_, table_path_, q,
                                                                   "AttentionLayer", &params);
    if (op != nullptr) {
        ctx.impl_params = params;
        if (!op->supports(ctx)) op = nullptr;   // the registry default instead (attention.cu:257-273)
    }
    if (op == nullptr) {
        params = Json::object();
        op = AttentionOpRegistry::instance().default_impl(ctx);
    }
    selected_[s] = op;
    selected_params_[s] = params;
    return op;
}

std::string AttentionLayer::selected_impl_id(ModelStage stage) const { return resolve_impl(stage)->impl_id(); }

void AttentionLayer::reset_operator_impl_cache() {
    selected_ = {nullptr, nullptr};
    selected_params_ = {Json::object(), Json::object()};
}

void AttentionLayer::check_tensor(const Tensor& t, const char* name) const {
    check_device(t, device_id_, name);
    check<ConfigurationError>(t.dtype() == dtype_, std::string(name) + " tensor dtype mismatch. Expected " +
                                                       dtype_name(dtype_) + ", got " + dtype_name(t.dtype()));
}

void AttentionLayer::forward_prefill(const Tensor& q, const Tensor& k, const Tensor& v, Tensor& o, bool causal,
                                     hipStream_t stream, uint32_t q_stride_n, uint32_t q_stride_h,
                                     uint32_t kv_stride_n, uint32_t kv_stride_h, uint32_t k_stride_n,
                                     uint32_t k_stride_h, bool k_already_prerotated, uint32_t q_rope_pos_offset,
                                     uint32_t k_rope_pos_offset) const {
    check_tensor(q, "q");
    check_tensor(k, "k");
    check_tensor(v, "v");
    check_tensor(o, "o");
    const auto &qs = q.shape(), &ks = k.shape(), &vs = v.shape(), &os = o.shape();
    check<InvalidRequestError>(qs.size() == 3 && (uint32_t)qs[1] == num_qo_heads_ && (uint32_t)qs[2] == head_dim_,
                               "q must have shape [qo_len, num_qo_heads, head_dim]");
    check<InvalidRequestError>(ks.size() == 3 && (uint32_t)ks[1] == num_kv_heads_ && (uint32_t)ks[2] == head_dim_,
                               "k must have shape [kv_len, num_kv_heads, head_dim]");
    check<InvalidRequestError>(vs.size() == 3 && vs[0] == ks[0] && (uint32_t)vs[1] == num_kv_heads_ &&
                                   (uint32_t)vs[2] == head_dim_,
                               "v must have shape [kv_len, num_kv_heads, head_dim]");
    check<InvalidRequestError>(os.size() == 3 && os[0] == qs[0] && (uint32_t)os[1] == num_qo_heads_ &&
                                   (uint32_t)os[2] == head_dim_,
                               "o must have shape [qo_len, num_qo_heads, head_dim]");
    AttentionOpContext ctx = base_ctx();
    ctx.q_stride_n = q_stride_n;
    ctx.q_stride_h = q_stride_h;
    ctx.kv_stride_n = kv_stride_n;
    ctx.kv_stride_h = kv_stride_h;
    ctx.k_stride_n = k_stride_n;
    ctx.k_stride_h = k_stride_h;
    ctx.q_rope_pos_offset = q_rope_pos_offset;
    ctx.k_rope_pos_offset = k_rope_pos_offset;
    ctx.k_already_prerotated = k_already_prerotated;
    AttentionOp* op = resolve_impl(ModelStage::Prefill);
    ctx.impl_params = selected_params_[0];
    op->forward_prefill(ctx, q, k, v, o, causal, stream);
}

void AttentionLayer::forward_decode(const Tensor& q, const Tensor& k, const Tensor& v, Tensor& o, hipStream_t stream,
                                    uint32_t* d_kv_len, uint32_t max_kv_len) const {
    check_tensor(q, "q");
    check_tensor(k, "k");
    check_tensor(v, "v");
    check_tensor(o, "o");
    const auto &qs = q.shape(), &ks = k.shape(), &vs = v.shape(), &os = o.shape();
    check<InvalidRequestError>(qs.size() == 3 && qs[0] == 1 && (uint32_t)qs[1] == num_qo_heads_ &&
                                   (uint32_t)qs[2] == head_dim_,
                               "In decode mode, q must have shape [1, num_qo_heads, head_dim]");
    check<InvalidRequestError>(ks.size() == 3 && (uint32_t)ks[1] == num_kv_heads_ && (uint32_t)ks[2] == head_dim_,
                               "k must have shape [kv_len, num_kv_heads, head_dim]");
    check<InvalidRequestError>(vs == ks, "v must have the shape of k");
    check<InvalidRequestError>(os == qs, "o must have shape [1, num_qo_heads, head_dim]");
    if (d_kv_len != nullptr) {
        check<InvalidRequestError>(max_kv_len > 0 && max_kv_len <= (uint32_t)ks[0],
                                   "max_kv_len must be in [1, k rows] with a device-side kv length");
    }
    AttentionOpContext ctx = base_ctx();
    AttentionOp* op = resolve_impl(ModelStage::Decode);
    ctx.impl_params = selected_params_[1];
    op->forward_decode(ctx, q, k, v, o, stream, d_kv_len, max_kv_len);
}

// =================================================================================
// RMSNormLayer
// =================================================================================
RMSNormLayer::RMSNormLayer(uint32_t layer_id, NormWeightType weight_type, const EngineConfig& cfg,
                           std::string layer_name)
    : model_name_(cfg.model_name()), hw_profile_(cfg.hw_profile()), table_path_(cfg.operator_table_path()),
      layer_name_(std::move(layer_name)), device_id_(cfg.device_id()), layer_id_(layer_id), weight_type_(weight_type) {
    role_ = weight_type == NormWeightType::Input           ? "input_norm"
            : weight_type == NormWeightType::PostAttention ? "post_attention_norm"
                                                           : "final_norm";
    hidden_ = cfg_u32(cfg.model_config(), "hidden_size", 4096);
    eps_ = (float)cfg.model_config().get_double("rms_norm_eps", 1e-6);
}

void RMSNormLayer::load_weights(const std::unordered_map<std::string, Tensor>& w) {
    std::string name;
    if (layer_id_ == UINT32_MAX || weight_type_ == NormWeightType::Final) name = "model.norm.weight";
    else if (weight_type_ == NormWeightType::Input)
        name = "model.layers." + std::to_string(layer_id_) + ".input_layernorm.weight";
    else name = "model.layers." + std::to_string(layer_id_) + ".post_attention_layernorm.weight";
    auto it = w.find(name);
    check<ConfigurationError>(it != w.end(), "RMSNorm weight not found for layer_id=" + std::to_string(layer_id_) +
                                                 ". Tried: " + name);
    const auto& s = it->second.shape();
    check<ConfigurationError>(s.size() == 1 && s[0] == (int64_t)hidden_,
                              "RMSNorm weight shape mismatch. Expected [" + std::to_string(hidden_) +
                                  "] for weight: " + name);
    weight_ = it->second;
    selected_ = {nullptr, nullptr};
}

NormOp* RMSNormLayer::resolve_impl(const RMSNormOpContext& ctx, ModelStage stage) {
    NormOp*& sel = selected_[slot_of(stage)];
    if (sel) return sel;
    OperatorQuery q;
    q.op_kind = "norm";
    q.layer_role = role_;
    q.op_name = "rms_norm";
    q.stage = stage_str(stage);
    NormOp* op = table_impl<NormOpRegistry, NormOp>(model_name_, hw_profile_, table_path_, q, "RMSNormLayer", nullptr);
    if (op != nullptr && !op->supports(ctx))
        throw ConfigurationError("RMSNormLayer: operator_impl_table selected unsupported impl '" + op->impl_id() + "'");
    if (op == nullptr) op = NormOpRegistry::instance().default_impl(ctx);
    sel = op;
    return op;
}

std::string RMSNormLayer::selected_impl_id(ModelStage stage) const {
    const NormOp* op = selected_[slot_of(stage)];
    return op ? op->impl_id() : "";
}

RMSNormOpContext RMSNormLayer::make_ctx(const Tensor& a, const char* name) const {
    check<ConfigurationError>(!weight_.empty(), "RMSNormLayer weight is not loaded");
    check_device(a, device_id_, name);
    const auto& s = a.shape();
    check<InvalidRequestError>(s.size() == 2 && s[1] == (int64_t)hidden_,
                               std::string(name) + " tensor must be [batch, " + std::to_string(hidden_) + "]");
    check<ConfigurationError>(a.dtype() == weight_.dtype(), std::string(name) + " dtype mismatch. Expected " +
                                                                dtype_name(weight_.dtype()) + ", got " +
                                                                dtype_name(a.dtype()));
    RMSNormOpContext c;
    c.batch_size = (uint32_t)s[0];
    c.hidden_size = hidden_;
    c.eps = eps_;
    c.dtype = weight_.dtype();
    return c;
}

void RMSNormLayer::forward_rmsnorm(const Tensor& input, Tensor& output, hipStream_t stream, ModelStage stage) {
    const RMSNormOpContext c = make_ctx(input, "Input");
    make_ctx(output, "Output");
    check<InvalidRequestError>(output.shape() == input.shape(), "Output tensor shape must equal the input's");
    resolve_impl(c, stage)->rms_norm_forward_fn()(c, input, weight_, output, stream);
}

void RMSNormLayer::forward_fused_add_rmsnorm(Tensor& inout, Tensor& residual, hipStream_t stream, ModelStage stage) {
    const RMSNormOpContext c = make_ctx(inout, "Inout");
    make_ctx(residual, "Residual");
    check<InvalidRequestError>(residual.shape() == inout.shape(), "Residual tensor shape must equal the inout's");
    resolve_impl(c, stage)->fused_add_rms_norm_forward_fn()(c, inout, residual, weight_, stream);
}

// =================================================================================
// ActivationLayer
// =================================================================================
ActivationLayer::ActivationLayer(const EngineConfig& cfg, std::string layer_name)
    : model_name_(cfg.model_name()), hw_profile_(cfg.hw_profile()), table_path_(cfg.operator_table_path()),
      layer_name_(std::move(layer_name)), device_id_(cfg.device_id()) {
    const Json& m = cfg.model_config();
    const uint32_t inter = cfg_u32(m, "intermediate_size", 0);
    hidden_ = inter != 0 ? inter : cfg_u32(m, "hidden_size", 4096);
    const std::string act = m.get_string("hidden_act", "silu");
    check<ConfigurationError>(act == "silu",
                              "Unsupported activation type: '" + act + "'. Currently only 'silu' is supported.");
}

void ActivationLayer::forward_silu_and_mul(const Tensor& input, Tensor& output, hipStream_t stream, ModelStage stage) {
    run(input, output, stream, stage, ActivationInputLayout::kGateUp);
}
void ActivationLayer::forward_silu_and_mul_up_gate(const Tensor& input, Tensor& output, hipStream_t stream,
                                                   ModelStage stage) {
    run(input, output, stream, stage, ActivationInputLayout::kUpGate);
}

std::string ActivationLayer::selected_impl_id(ModelStage stage) const {
    const ActivationOp* op = selected_[slot_of(stage)];
    return op ? op->impl_id() : "";
}

void ActivationLayer::run(const Tensor& input, Tensor& output, hipStream_t stream, ModelStage stage,
                          ActivationInputLayout layout) {
    check_device(input, device_id_, "Input");
    check_device(output, device_id_, "Output");
    const auto &is = input.shape(), &os = output.shape();
    check<InvalidRequestError>(is.size() >= 2, "Input tensor must have at least 2 dimensions");
    check<InvalidRequestError>(is.back() == 2 * (int64_t)hidden_,
                               "Input tensor last dimension mismatch. Expected " + std::to_string(2 * hidden_) +
                                   " (2 * hidden_size from config: " + std::to_string(hidden_) + "), got " +
                                   std::to_string(is.back()));
    check<InvalidRequestError>(os.size() == is.size(), "Output tensor must have the same number of dimensions as input");
    for (size_t i = 0; i + 1 < os.size(); ++i)
        check<InvalidRequestError>(os[i] == is[i], "Output tensor shape mismatch at dimension " + std::to_string(i));
    check<InvalidRequestError>(os.back() == (int64_t)hidden_, "Output tensor last dimension mismatch. Expected " +
                                                                  std::to_string(hidden_));
    check<InvalidRequestError>(input.dtype() == output.dtype(), "Input and output tensors must have the same dtype");
    ActivationOpContext c;
    c.batch_size = std::accumulate(is.begin(), is.end() - 1, (int64_t)1, std::multiplies<int64_t>());
    c.hidden_size = hidden_;
    c.dtype = input.dtype();
    c.kind = ActivationKind::kSilu;
    c.input_layout = layout;
    ActivationOp*& sel = selected_[slot_of(stage)];
    if (sel == nullptr) {
        OperatorQuery q;
        q.op_kind = "activation";
        q.layer_role = "mlp_activation";
        q.op_name = "silu_and_mul";
        q.stage = stage_str(stage);
        ActivationOp* op = table_impl<ActivationOpRegistry, ActivationOp>(model_name_, hw_profile_, table_path_, q,
                                                                          "ActivationLayer", nullptr);
        if (op != nullptr && !op->supports(c))
            throw ConfigurationError("ActivationLayer: operator_impl_table selected unsupported impl '" +
                                     op->impl_id() + "'");
        sel = op ? op : ActivationOpRegistry::instance().default_impl(c);
    }
    sel->act_and_mul(c, input, output, stream);
}

// =================================================================================
// SamplerLayer
// =================================================================================
SamplerLayer::SamplerLayer(const EngineConfig& cfg) : device_id_(cfg.device_id()) {
    vocab_ = cfg_u32(cfg.model_config(), "vocab_size", 32000);
    temperature_ = cfg.temperature();
    top_p_ = cfg.top_p();
    seed_ = cfg.seed();
    check<ConfigurationError>(temperature_ >= 0.0f,
                              "temperature must be non-negative. Got: " + std::to_string(temperature_));
    check<ConfigurationError>(top_p_ > 0.0f, "top_p must be positive. Got: " + std::to_string(top_p_));
}

void SamplerLayer::forward_sampling(const Tensor& logits, Tensor& token_ids, hipStream_t stream) {
    check_device(logits, device_id_, "Logits");
    check_device(token_ids, device_id_, "Token IDs");
    const auto& ls = logits.shape();
    check<InvalidRequestError>(ls.size() == 2, "Logits tensor must be 2D [batch_size, vocab_size]. Got " +
                                                   std::to_string(ls.size()) + "D");
    check<InvalidRequestError>(ls[1] == (int64_t)vocab_, "Vocab size mismatch. Expected " + std::to_string(vocab_) +
                                                             ", got " + std::to_string(ls[1]));
    const int64_t rows = ls[0];
    check<InvalidRequestError>(token_ids.shape().size() == 1 && token_ids.shape()[0] == rows,
                               "Token IDs tensor shape mismatch. Expected [" + std::to_string(rows) + "]");
    check<InvalidRequestError>(token_ids.dtype() == DType::Int32, "Token IDs tensor dtype must be Int32");
    check<InvalidRequestError>(logits.dtype() == DType::Float32, "Logits dtype must be Float32");
    const float* lg = static_cast<const float*>(logits.data_ptr());
    int32_t* out = static_cast<int32_t*>(token_ids.data_ptr());
    if (temperature_ < 1e-6f) {
        const size_t need = efm_sampler_greedy_workspace_bytes(rows, vocab_);
        Tensor ws = cache_buf("greedy_sampler_ws", need, device_id_);
        efm_check(efm_sampler_greedy(rows, vocab_, lg, out, ws.data_ptr(), ws.nbytes(), stream), "greedy sampling");
        return;
    }
    const size_t need = efm_sampler_top_p_workspace_bytes(vocab_);
    Tensor ws = cache_buf("sampler_top_p_ws", need, device_id_);
    for (int64_t r = 0; r < rows; ++r)
        efm_check(efm_sampler_top_p(vocab_, lg + r * (int64_t)vocab_, temperature_, top_p_, seed_, (uint64_t)r,
                                    nullptr, out + r, ws.data_ptr(), ws.nbytes(), stream),
                  "sampling");
}

// =================================================================================
// EmbedHeadLayer
// =================================================================================
EmbedHeadLayer::EmbedHeadLayer(const EngineConfig& cfg, std::string) : device_id_(cfg.device_id()) {
    vocab_ = cfg_u32(cfg.model_config(), "vocab_size", 32000);
    hidden_ = cfg_u32(cfg.model_config(), "hidden_size", 4096);
}

void EmbedHeadLayer::load_weights(const std::unordered_map<std::string, Tensor>& w) {
    auto it = w.find("model.embed_tokens.weight");
    check<ConfigurationError>(it != w.end(), "EmbedHeadLayer: missing 'model.embed_tokens.weight' in prefill_weights");
    const auto& s = it->second.shape();
    check<ConfigurationError>(s.size() == 2, "EmbedHeadLayer: embedding table must be 2D [vocab_size, hidden_size]");
    check<ConfigurationError>(s[0] == (int64_t)vocab_, "EmbedHeadLayer: embedding table vocab_size mismatch. Expected " +
                                                           std::to_string(vocab_) + ", got " + std::to_string(s[0]));
    check<ConfigurationError>(s[1] == (int64_t)hidden_,
                              "EmbedHeadLayer: embedding table hidden_size mismatch. Expected " +
                                  std::to_string(hidden_) + ", got " + std::to_string(s[1]));
    check<ConfigurationError>(it->second.dtype() == DType::BFloat16,
                              "EmbedHeadLayer: embedding table dtype must be BFloat16 on this build");
    table_ = it->second;
}

void EmbedHeadLayer::check_ids_out(const Tensor& ids, const Tensor& out) const {
    check<ConfigurationError>(!table_.empty(), "EmbedHeadLayer weights are not loaded");
    check_device(ids, device_id_, "Input token_ids");
    check_device(out, device_id_, "Output");
    const auto& ts = ids.shape();
    check<InvalidRequestError>(ts.size() == 2, "Token IDs tensor must be 2D [batch_size, seq_len]. Got " +
                                                   std::to_string(ts.size()) + "D");
    check<InvalidRequestError>(ids.dtype() == DType::Int32, "Token IDs dtype must be Int32");
    const auto& os = out.shape();
    check<InvalidRequestError>(os.size() == 3 && os[0] == ts[0] && os[1] == ts[1] && os[2] == (int64_t)hidden_,
                               "Output tensor must be [batch_size, seq_len, " + std::to_string(hidden_) + "]");
    check<InvalidRequestError>(out.dtype() == table_.dtype(), "Output dtype must match embedding table dtype");
}

void EmbedHeadLayer::forward_for_tokens(const Tensor& ids, Tensor& out, hipStream_t stream) {
    check_ids_out(ids, out);
    const int64_t n = ids.shape()[0] * ids.shape()[1];
    efm_check(efm_embedding_lookup(n, hidden_, vocab_, static_cast<const int32_t*>(ids.data_ptr()), table_.data_ptr(),
                                   nullptr, 0, -1, out.data_ptr(), stream),
              "embedding lookup");
}

void EmbedHeadLayer::forward_for_embeddings(const Tensor& ids, const Tensor& embeddings, Tensor& out,
                                            int32_t embed_token_id, hipStream_t stream) {
    check_ids_out(ids, out);
    check_device(embeddings, device_id_, "Input embeddings");
    const auto& es = embeddings.shape();
    check<InvalidRequestError>(es.size() == 2 && es[1] == (int64_t)hidden_,
                               "Embeddings tensor must be 2D [num_custom_embeddings, " + std::to_string(hidden_) + "]");
    check<InvalidRequestError>(embeddings.dtype() == table_.dtype(), "Embeddings dtype must match embedding table dtype");
    if (embed_token_id >= 0)
        check<InvalidRequestError>((int64_t)embed_token_id + es[0] <= (int64_t)INT32_MAX,
                                   "embed_token_id + num_custom_embeddings exceeds int32_t max value");
    const int64_t n = ids.shape()[0] * ids.shape()[1];
    efm_check(efm_embedding_lookup(n, hidden_, vocab_, static_cast<const int32_t*>(ids.data_ptr()), table_.data_ptr(),
                                   embeddings.data_ptr(), es[0], embed_token_id, out.data_ptr(), stream),
              "embedding lookup");
}

// =================================================================================
// LMHeadLinearLayer
// =================================================================================
LMHeadLinearLayer::LMHeadLinearLayer(const std::string& prefix, const EngineConfig& cfg, uint32_t in, uint32_t out,
                                     std::string layer_name)
    : LinearLayer(prefix, cfg, in, out, std::move(layer_name)), device_id_(cfg.device_id()) {}

void LMHeadLinearLayer::load_weights(const std::unordered_map<std::string, Tensor>& w) {
    const std::vector<std::string> names = {layer_prefix() + ".weight", "model." + layer_prefix() + ".weight",
                                            "model.embed_tokens.weight"};
    for (const auto& n : names) {
        auto it = w.find(n);
        if (it != w.end()) {
            LinearLayer::load_weights(it->second, nullptr);
            return;
        }
    }
    throw ConfigurationError("LMHeadLinearLayer: none of [" + names[0] + ", " + names[1] + ", " + names[2] +
                             "] found in prefill_weights");
}

bool LMHeadLinearLayer::try_forward_top1(const Tensor& input, Tensor& token_out, hipStream_t stream,
                                         ModelStage stage) {
    if (stage != ModelStage::Decode) return false;
    const Tensor* w = weight_tensor(ModelStage::Decode);
    check<InvalidRequestError>(w != nullptr && w->data_ptr() != nullptr, "LMHeadLinearLayer is not initialized");
    if (bias_tensor(ModelStage::Decode) != nullptr) return false;
    const auto &is = input.shape(), &ts = token_out.shape();
    check<InvalidRequestError>(is.size() == 2 && is[0] == 1 && is[1] == (int64_t)in_features(),
                               "LMHeadLinearLayer::try_forward_top1 expects input shape [1, hidden_size]");
    check<InvalidRequestError>(ts.size() == 1 && ts[0] == 1,
                               "LMHeadLinearLayer::try_forward_top1 expects token_out shape [1]");
    check<InvalidRequestError>(token_out.dtype() == DType::Int32,
                               "LMHeadLinearLayer::try_forward_top1 expects token_out dtype Int32");
    if (input.dtype() != DType::BFloat16 || w->dtype() != DType::BFloat16) return false;
    check_device(input, device_id_, "Input");
    check_device(token_out, device_id_, "Token");
    const size_t need = efm_lm_head_top1_workspace_bytes(out_features());
    Tensor ws = cache_buf("lm_head_top1_workspace", need, device_id_);
    efm_check(efm_lm_head_top1(in_features(), out_features(), input.data_ptr(), w->data_ptr(),
                               static_cast<int32_t*>(token_out.data_ptr()), ws.data_ptr(), ws.nbytes(), stream),
              "LMHeadLinearLayer::try_forward_top1");
    return true;
}

// =================================================================================
// Fused projections: weights and the fused SwiGLU entry points
// =================================================================================
namespace {
const Tensor* find_w(const std::unordered_map<std::string, Tensor>& w, const std::string& n) {
    auto it = w.find(n);
    return it == w.end() ? nullptr : &it->second;
}

// Biases of `parts` rows each, concatenated; a missing part contributes zeros.
Tensor concat_bias(const std::vector<const Tensor*>& biases, const std::vector<uint32_t>& rows, int32_t device_id,
                   hipStream_t s) {
    const int64_t total = std::accumulate(rows.begin(), rows.end(), (int64_t)0);
    Tensor out = Tensor::zeros({total}, DType::BFloat16, Device::GPU, device_id);
    size_t off = 0;
    for (size_t i = 0; i < biases.size(); ++i) {
        if (biases[i] != nullptr) {
            check<ModelNotLoadedError>(biases[i]->numel() == rows[i] && biases[i]->dtype() == DType::BFloat16,
                                       "fused projection bias shape or dtype mismatch");
            hip_check(hipMemcpyAsync(static_cast<char*>(out.data_ptr()) + off, biases[i]->data_ptr(),
                                     biases[i]->nbytes(), hipMemcpyDeviceToDevice, s),
                      "fuse bias");
        }
        off += (size_t)rows[i] * 2;
    }
    return out;
}
}  // namespace

void load_fused_qkv_weights(FusedQKVLinearLayer& layer, const std::string& base,
                            const std::unordered_map<std::string, Tensor>& w, uint32_t q_out, uint32_t k_out,
                            uint32_t v_out, int32_t device_id) {
    if (const Tensor* fw = find_w(w, base + ".qkv_fused.weight")) {
        layer.load_weights(*fw, find_w(w, base + ".qkv_fused.bias"));
        return;
    }
    const char* parts[3] = {".q_proj", ".k_proj", ".v_proj"};
    const uint32_t rows[3] = {q_out, k_out, v_out};
    std::vector<const Tensor*> ws, bs;
    for (int i = 0; i < 3; ++i) {
        const Tensor* t = find_w(w, base + parts[i] + ".weight");
        check<ConfigurationError>(t != nullptr, "FusedQKVLinearLayer: missing " + base + parts[i] + ".weight");
        check<ConfigurationError>(t->shape().size() == 2 && t->shape()[0] == rows[i],
                                  "FusedQKVLinearLayer: " + base + parts[i] + ".weight has the wrong row count");
        ws.push_back(t);
        bs.push_back(find_w(w, base + parts[i] + ".bias"));
    }
    hip_check(hipSetDevice(device_id), "hipSetDevice");
    Tensor fw = concat_rows(ws, device_id, nullptr);
    const bool any_bias = bs[0] || bs[1] || bs[2];
    Tensor fb = any_bias ? concat_bias(bs, {q_out, k_out, v_out}, device_id, nullptr) : Tensor();
    hip_check(hipStreamSynchronize(nullptr), "fuse qkv");
    layer.load_weights(fw, any_bias ? &fb : nullptr);
    WeightLoader::instance().register_tensor(ModelStage::Prefill, base + ".qkv_fused.weight", fw);
    if (any_bias) WeightLoader::instance().register_tensor(ModelStage::Prefill, base + ".qkv_fused.bias", fb);
}

void load_fused_gate_up_weights(FusedGateUpLinearLayer& layer, const std::string& base,
                                const std::unordered_map<std::string, Tensor>& w, int32_t device_id) {
    if (const Tensor* fw = find_w(w, base + ".gate_up_fused.weight")) {
        layer.load_weights(*fw, find_w(w, base + ".gate_up_fused.bias"));
        return;
    }
    const Tensor* up = find_w(w, base + ".up_proj.weight");
    const Tensor* gate = find_w(w, base + ".gate_proj.weight");
    check<ConfigurationError>(up != nullptr && gate != nullptr,
                              "FusedGateUpLinearLayer: missing " + base + ".up_proj.weight or .gate_proj.weight");
    check<ConfigurationError>(up->shape().size() == 2 && up->shape()[0] == layer.up_out_features() &&
                                  gate->shape().size() == 2 && gate->shape()[0] == layer.gate_out_features(),
                              "FusedGateUpLinearLayer: projection row counts do not match the layer");
    const Tensor* ub = find_w(w, base + ".up_proj.bias");
    const Tensor* gb = find_w(w, base + ".gate_proj.bias");
    hip_check(hipSetDevice(device_id), "hipSetDevice");
    Tensor fw = concat_rows({up, gate}, device_id, nullptr);
    const bool any_bias = ub || gb;
    Tensor fb = any_bias ? concat_bias({ub, gb}, {layer.up_out_features(), layer.gate_out_features()}, device_id,
                                       nullptr)
                         : Tensor();
    hip_check(hipStreamSynchronize(nullptr), "fuse gate/up");
    layer.load_weights(fw, any_bias ? &fb : nullptr);
    WeightLoader::instance().register_tensor(ModelStage::Prefill, base + ".gate_up_fused.weight", fw);
    if (any_bias) WeightLoader::instance().register_tensor(ModelStage::Prefill, base + ".gate_up_fused.bias", fb);
}

FusedGateUpLinearLayer::FusedGateUpLinearLayer(const std::string& hf_mlp_prefix, const EngineConfig& cfg,
                                               uint32_t hidden, uint32_t gate_out_features, uint32_t up_out_features,
                                               std::string layer_name)
    : LinearLayer(hf_mlp_prefix, "fused_gate_up", cfg, hidden, gate_out_features + up_out_features,
                  std::move(layer_name)),
      gate_out_(gate_out_features), up_out_(up_out_features), model_name_(cfg.model_name()),
      hw_profile_(cfg.hw_profile()), table_path_(cfg.operator_table_path()) {}

bool FusedGateUpLinearLayer::try_forward_decode_swiglu_fused(const Tensor& input, Tensor& output, hipStream_t stream) {
    const auto &is = input.shape(), &os = output.shape();
    if (is.size() != 2 || os.size() != 2 || is[0] != 1 || os[0] != 1) return false;
    if (is[1] != (int64_t)in_features() || os[1] != (int64_t)up_out_) return false;
    return try_forward_swiglu_fused_impl(input, output, ModelStage::Decode, stream);
}

bool FusedGateUpLinearLayer::try_forward_prefill_swiglu_fused(const Tensor& input, Tensor& output,
                                                              hipStream_t stream) {
    const auto &is = input.shape(), &os = output.shape();
    if (is.size() != 2 || os.size() != 2 || is[0] < 64 || os[0] != is[0]) return false;
    if (is[1] != (int64_t)in_features() || os[1] != (int64_t)up_out_) return false;
    return try_forward_swiglu_fused_impl(input, output, ModelStage::Prefill, stream);
}

bool FusedGateUpLinearLayer::try_forward_swiglu_fused_impl(const Tensor& input, Tensor& output, ModelStage stage,
                                                           hipStream_t stream) {
    const Tensor* w = weight_tensor(stage);
    if (w == nullptr || w->data_ptr() == nullptr || bias_tensor(stage) != nullptr) return false;
    if (gate_out_ != up_out_ || input.dtype() != DType::BFloat16 || output.dtype() != DType::BFloat16) return false;
    FusedGateUpActivationContext c;
    c.stage = stage;
    c.m = input.shape()[0];
    c.hidden = in_features();
    c.intermediate = up_out_;
    OperatorQuery q;
    q.op_kind = "fused_gate_up_activation";
    q.layer_role = "fused_gate_up";
    q.op_name = layer_prefix();
    q.stage = stage_str(stage);
    LinearShapeSignature sig;
    sig.m = (int32_t)c.m;
    sig.in_features = in_features();
    sig.out_features = out_features();
    q.shape_sig = sig.to_string();
    FusedGateUpActivationOp* op = table_impl<FusedGateUpActivationRegistry, FusedGateUpActivationOp>(
        model_name_, hw_profile_, table_path_, q, "FusedGateUpLinearLayer", nullptr);
    if (op != nullptr && !op->supports(c))
        throw ConfigurationError("FusedGateUpLinearLayer: operator_impl_table selected unsupported impl '" +
                                 op->impl_id() + "'");
    if (op == nullptr) op = FusedGateUpActivationRegistry::instance().default_impl(c);
    if (op == nullptr || !op->prepare(c, *w).available) return false;
    check_device(input, w->device().second, "Input");
    check_device(output, w->device().second, "Output");
    return op->run(c, *w, input, output, stream);
}

}  // namespace edge_fm
