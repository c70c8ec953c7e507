// Operator layer of the MI355X runtime: the reference's operator interfaces
// (src/operators/*.h, src/layers/linear.h:110-153), their registries and the
// operator implementation table, with gfx950 implementations that call the
// edgefm_hip C ABI.
#pragma once

#include <map>
#include <memory>
#include <mutex>
#include <tuple>
#include <optional>
#include <string>
#include <unordered_map>
#include <vector>

#include "core.hpp"
#include "json.hpp"

namespace edge_fm {

// ---------------------------------------------------------------------------------
// Operator implementation table (src/operators/operator_impl_table.h:13-66). Same
// record schema ("edgefm_operator_impl_table_v1") and the same resolution rule:
// per-field exact-or-wildcard matching with weights op_name 1e6, layer_role 1e5,
// shape_sig 1e4, stage 1e3, hw_profile 200 exact / 120 prefix, model 100, op_kind 10;
// the last of equally scored records wins.
// ---------------------------------------------------------------------------------
struct OperatorImplRecord {
    std::string model_name, hw_profile, op_kind, layer_role, op_name, stage, shape_sig, impl_id;
    Json impl_params = Json::object();

    Json to_json() const;
    static OperatorImplRecord from_json(const Json& j);
};

struct OperatorQuery {
    std::string op_kind, layer_role, op_name, stage, shape_sig;
};

std::string normalize_identifier(const std::string& raw);
std::string normalize_model_name(const std::string& raw);

class OperatorImplTable {
public:
    static OperatorImplTable& instance();
    std::optional<OperatorImplRecord> resolve(const std::string& model_name, const std::string& hw_profile,
                                              const std::string& table_path, const OperatorQuery& q);
    std::vector<OperatorImplRecord> all_records(const std::string& table_path);
    void invalidate(const std::string& table_path);

private:
    const std::vector<OperatorImplRecord>& load_locked(const std::string& table_path);
    std::mutex mu_;
    std::unordered_map<std::string, std::vector<OperatorImplRecord>> tables_;
};

// ---------------------------------------------------------------------------------
// Attention (src/operators/attention_op.h:15-96)
// ---------------------------------------------------------------------------------
enum class AttentionPosEncoding { kNone, kRoPELlama };

struct AttentionOpContext {
    uint32_t num_qo_heads = 0, num_kv_heads = 0, head_dim = 0;
    uint32_t q_stride_n = 0, q_stride_h = 0, k_stride_n = 0, k_stride_h = 0, kv_stride_n = 0, kv_stride_h = 0;
    float rope_scale = 1.0f, rope_theta = 1000000.0f;
    uint32_t q_rope_pos_offset = 0, k_rope_pos_offset = 0;
    DType dtype = DType::BFloat16;
    AttentionPosEncoding pos_encoding = AttentionPosEncoding::kRoPELlama;
    bool k_already_prerotated = false;
    int32_t device_id = 0;
    Json impl_params = Json::object();
    // Decode planning facts (not in the reference's context; 0 = unknown): the model's
    // hidden size and the longest cache a decode step reads. The fused decode impls
    // support a shape only when both are known.
    uint32_t decode_hidden = 0, decode_max_kv_len = 0;
};

efm_attention_ctx to_c_ctx(const AttentionOpContext& c);
// "num_qo_heads=<n>|num_kv_heads=<n>|head_dim=<n>" (src/layers/attention.cu:149-153)
std::string attention_shape_sig(uint32_t num_qo_heads, uint32_t num_kv_heads, uint32_t head_dim);

class AttentionOp {
public:
    virtual ~AttentionOp() = default;
    virtual std::string impl_id() const = 0;
    virtual bool supports(const AttentionOpContext& ctx) const = 0;
    virtual void forward_prefill(const AttentionOpContext& ctx, const Tensor& q, const Tensor& k, const Tensor& v,
                                 Tensor& o, bool causal, hipStream_t stream) = 0;
    virtual void forward_decode(const AttentionOpContext& ctx, const Tensor& q, const Tensor& k, const Tensor& v,
                                Tensor& o, hipStream_t stream, uint32_t* d_kv_len, uint32_t max_kv_len) = 0;
};

class AttentionOpRegistry {
public:
    static AttentionOpRegistry& instance();
    AttentionOp* find_impl_by_id(const std::string& id) const;
    AttentionOp* default_impl(const AttentionOpContext& ctx) const;

private:
    AttentionOpRegistry();
    std::vector<std::unique_ptr<AttentionOp>> impls_;
};

// ---------------------------------------------------------------------------------
// RMSNorm (src/operators/norm_op.h:14-82)
// ---------------------------------------------------------------------------------
struct RMSNormOpContext {
    uint32_t batch_size = 0, hidden_size = 0;
    float eps = 1e-6f;
    DType dtype = DType::BFloat16;
};

using RMSNormForwardFn = void (*)(const RMSNormOpContext&, const Tensor& input, const Tensor& weight, Tensor& output,
                                  hipStream_t);
using FusedAddRMSNormForwardFn = void (*)(const RMSNormOpContext&, Tensor& inout, Tensor& residual,
                                          const Tensor& weight, hipStream_t);

class NormOp {
public:
    virtual ~NormOp() = default;
    virtual std::string impl_id() const = 0;
    virtual bool supports(const RMSNormOpContext& ctx) const = 0;
    virtual RMSNormForwardFn rms_norm_forward_fn() const = 0;
    virtual FusedAddRMSNormForwardFn fused_add_rms_norm_forward_fn() const = 0;
};

class NormOpRegistry {
public:
    static NormOpRegistry& instance();
    NormOp* find_impl_by_id(const std::string& id) const;
    NormOp* default_impl(const RMSNormOpContext& ctx) const;

private:
    NormOpRegistry();
    std::vector<std::unique_ptr<NormOp>> impls_;
};

// ---------------------------------------------------------------------------------
// Activation (src/operators/activation_op.h:14-61)
// ---------------------------------------------------------------------------------
enum class ActivationKind { kSilu };
enum class ActivationInputLayout { kGateUp, kUpGate };

struct ActivationOpContext {
    int64_t batch_size = 0, hidden_size = 0;
    DType dtype = DType::BFloat16;
    ActivationKind kind = ActivationKind::kSilu;
    ActivationInputLayout input_layout = ActivationInputLayout::kGateUp;
};

class ActivationOp {
public:
    virtual ~ActivationOp() = default;
    virtual std::string impl_id() const = 0;
    virtual bool supports(const ActivationOpContext& ctx) const = 0;
    virtual void act_and_mul(const ActivationOpContext& ctx, const Tensor& input, Tensor& output,
                             hipStream_t stream) = 0;
};

class ActivationOpRegistry {
public:
    static ActivationOpRegistry& instance();
    ActivationOp* find_impl_by_id(const std::string& id) const;
    ActivationOp* default_impl(const ActivationOpContext& ctx) const;

private:
    ActivationOpRegistry();
    std::vector<std::unique_ptr<ActivationOp>> impls_;
};

// ---------------------------------------------------------------------------------
// Linear: LinearLayer with the reference's nested interface types (WeightSet,
// LinearShapeSignature, LinearOpContext, CachedDescriptors, LinearImpl with prepare /
// forward: src/layers/linear.h:100-153) and LinearOpRegistry (src/operators/
// linear_registry.h:9-24). The impl for (stage, m) is resolved once from the operator
// table (op_kind linear, layer_role from the prefix, op_name = the prefix, stage,
// shape_sig = LinearShapeSignature::to_string) exactly as LinearLayer::resolve_impl does
// (src/operators/linear_impl.cu:866-915): a table record naming an unknown or unsupporting
// impl is a ConfigurationError; without a record the registry default runs.
// ---------------------------------------------------------------------------------
class EngineConfig;
class PrefillLinearSourceOp;

// "fused_qkv" (…qkv_fused), "fused_gate_up" (…gate_up_fused), "attention_output"
// (….o_proj), "mlp_down" (….down_proj), "lm_head", else "linear"
// (src/layers/linear.cu:41-58).
std::string infer_layer_role(const std::string& layer_prefix);
std::string stage_key(ModelStage stage);

class LinearLayer {
public:
    enum class QuantType { FP16_BF16, INT4_GROUPWISE, INT8, FP4 };

    struct WeightSet {
        QuantType quant_type_ = QuantType::FP16_BF16;
        const Tensor* weight_ = nullptr;           // [out_features, in_features]
        const Tensor* bias_ = nullptr;             // [out_features] or null
        const Tensor* scaling_factors_ = nullptr;  // quantized weights only (none supported here)
        uint32_t group_size_ = 128;
    };

    struct LinearShapeSignature {
        int32_t m = -1;
        DType input_dtype = DType::BFloat16, weight_dtype = DType::BFloat16, output_dtype = DType::BFloat16;
        uint32_t in_features = 0, out_features = 0;
        // "m=<m>|input=<dtype>|weight=<dtype>|output=<dtype>|in_features=<k>|out_features=<n>"
        std::string to_string() const;
    };

    struct LinearOpContext {
        std::string layer_prefix, layer_role;
        ModelStage stage = ModelStage::Prefill;
        LinearShapeSignature shape;
        bool has_bias = false;
    };

    // Per (stage, m) state an impl keeps between calls: the resolved impl and, for the
    // MFMA GEMM, the split-K scratch its plan for this shape needs.
    struct CachedDescriptors {
        std::string selected_impl_id_;
        Json selected_impl_params_ = Json::object();
        size_t workspace_bytes_ = 0;
        Tensor workspace_;
        bool prepared_ = false;
    };

    class LinearImpl {
    public:
        virtual ~LinearImpl() = default;
        virtual std::string impl_id() const = 0;
        virtual bool supports(const LinearOpContext& ctx, const WeightSet& weight_set) const = 0;
        virtual void prepare(LinearLayer& owner, const LinearOpContext& ctx, const WeightSet& weight_set,
                             const Tensor& input, Tensor& output, hipStream_t stream, CachedDescriptors& cached) = 0;
        virtual void forward(LinearLayer& owner, const LinearOpContext& ctx, const WeightSet& weight_set,
                             const Tensor& input, Tensor& output, hipStream_t stream, CachedDescriptors& cached) = 0;
    };

    LinearLayer(const std::string& layer_prefix, const EngineConfig& engine_config, uint32_t in_features,
                uint32_t out_features, std::string layer_name = "");
    ~LinearLayer();
    LinearLayer(const LinearLayer&) = delete;
    LinearLayer& operator=(const LinearLayer&) = delete;

    // The layer's weight [out, in] (+ bias [out]); prefill and decode share it (the
    // engine loads one checkpoint for both stages).
    void load_weights(const Tensor& weight, const Tensor* bias);
    // output[m, out] = input[m, in] . W^T (+ bias) through the impl resolved for (stage, m).
    void forward_fp16_bf16(const Tensor& input, Tensor& output, hipStream_t stream = nullptr,
                           ModelStage stage = ModelStage::Prefill);
    // The impl forward_fp16_bf16 runs for (stage, m, output dtype), resolved without running.
    std::string selected_impl_id(ModelStage stage, int32_t m, DType output_dtype = DType::BFloat16);
    LinearImpl* resolve_impl(const LinearOpContext& ctx, const WeightSet& weight_set, CachedDescriptors& cached) const;
    void reset_operator_impl_cache();

    const Tensor* weight_tensor(ModelStage stage = ModelStage::Prefill) const;
    const Tensor* bias_tensor(ModelStage stage = ModelStage::Prefill) const;
    const std::string& layer_prefix() const { return prefix_; }
    const std::string& layer_role() const { return role_; }
    const std::string& layer_name() const { return name_; }
    uint32_t in_features() const { return in_; }
    uint32_t out_features() const { return out_; }
    PrefillLinearSourceOp* prefill_linear_source_op() const { return source_op_.get(); }

protected:
    // explicit role (the fused subclasses: their prefixes carry no role suffix)
    LinearLayer(const std::string& layer_prefix, std::string layer_role, const EngineConfig& engine_config,
                uint32_t in_features, uint32_t out_features, std::string layer_name);

private:
    LinearOpContext make_ctx(int32_t m, DType input_dtype, DType output_dtype, ModelStage stage) const;
    CachedDescriptors& cache_slot(ModelStage stage, int32_t m, DType output_dtype);

    std::string prefix_, role_, name_;
    std::string model_name_, hw_profile_, table_path_;
    uint32_t in_ = 0, out_ = 0;
    Tensor weight_, bias_;
    WeightSet ws_;
    std::map<std::tuple<int, int32_t, int>, CachedDescriptors> cache_;
    std::unique_ptr<PrefillLinearSourceOp> source_op_;
};

// Fused [Q; K; V] rows with [bq; bk; bv] under the attention prefix
// (model.layers.<l>.self_attn, role fused_qkv: src/layers/linear.h FusedQKVLinearLayer).
class FusedQKVLinearLayer : public LinearLayer {
public:
    FusedQKVLinearLayer(const std::string& hf_attn_prefix, const EngineConfig& engine_config, uint32_t hidden,
                        uint32_t q_dim, uint32_t k_dim, uint32_t v_dim, std::string layer_name = "")
        : LinearLayer(hf_attn_prefix, "fused_qkv", engine_config, hidden, q_dim + k_dim + v_dim,
                      std::move(layer_name)) {}
};

// Fused [up; gate] rows under the MLP prefix (model.layers.<l>.mlp, role fused_gate_up:
// src/layers/linear.h FusedGateUpLinearLayer; rows [0, I) up, [I, 2 I) gate).
class FusedGateUpLinearLayer : public LinearLayer {
public:
    FusedGateUpLinearLayer(const std::string& hf_mlp_prefix, const EngineConfig& engine_config, uint32_t hidden,
                           uint32_t gate_out_features, uint32_t up_out_features, std::string layer_name = "");
    // output [m, I] = silu(x . Wgate^T) * (x . Wup^T) in one fused launch, through the
    // fused gate/up + SwiGLU op resolved for (stage, the layer prefix, m) from the operator
    // table (linear.cu:2054-2223: a record naming an unknown or unsupporting impl is a
    // ConfigurationError). Returns false, having done nothing, when the shapes are not
    // decode [1, H] -> [1, I] (prefill: m >= 64) or no impl supports them.
    bool try_forward_decode_swiglu_fused(const Tensor& input, Tensor& output, hipStream_t stream);
    bool try_forward_prefill_swiglu_fused(const Tensor& input, Tensor& output, hipStream_t stream);
    uint32_t gate_out_features() const { return gate_out_; }
    uint32_t up_out_features() const { return up_out_; }

private:
    bool try_forward_swiglu_fused_impl(const Tensor& input, Tensor& output, ModelStage stage, hipStream_t stream);
    uint32_t gate_out_ = 0, up_out_ = 0;
    std::string model_name_, hw_profile_, table_path_;
};

class LinearOpRegistry {
public:
    static LinearOpRegistry& instance();
    LinearLayer::LinearImpl* find_impl_by_id(const std::string& id) const;
    LinearLayer::LinearImpl* default_impl(const LinearLayer::LinearOpContext& ctx,
                                          const LinearLayer::WeightSet& weight_set) const;

private:
    LinearOpRegistry();
    std::vector<std::unique_ptr<LinearLayer::LinearImpl>> impls_;
};

// ---------------------------------------------------------------------------------
// Prefill source ops (src/operators/prefill_linear_source_op.h:16-23,
// prefill_mlp_source_op.h:13-20): try_forward runs the projection (or the whole MLP:
// gate/up GEMM with its SwiGLU epilogue, then down) on this library's MFMA kernels and
// returns true, or returns false, having done nothing, when the shape or dtypes are not
// ones it handles; the caller then takes its layered path. Each keeps the scratch its
// kernels need per shape until reset_runtime_caches().
// ---------------------------------------------------------------------------------
class PrefillLinearSourceOp {
public:
    explicit PrefillLinearSourceOp(const EngineConfig& config);
    ~PrefillLinearSourceOp();
    bool try_forward(const std::string& role, int32_t layer_id, const Tensor& input, const Tensor& weight,
                     const Tensor* bias, Tensor& output, hipStream_t stream);
    void reset_runtime_caches();

private:
    int32_t device_id_ = 0;
};

class PrefillMlpSourceOp {
public:
    explicit PrefillMlpSourceOp(const EngineConfig& config);
    ~PrefillMlpSourceOp();
    // gate_up_weight [2 I, H] in the fused [up; gate] layout, down_weight [H, I];
    // input [m, H] -> output [m, H]
    bool try_forward(int32_t layer_id, const Tensor& input, const Tensor& gate_up_weight, const Tensor& down_weight,
                     Tensor& output, hipStream_t stream);
    void reset_runtime_caches();
    // Changes whenever the intermediate buffer is replaced (captured work that used the
    // old one must be captured again).
    uint64_t generation() const { return generation_; }

private:
    int32_t device_id_ = 0;
    Tensor intermediate_;   // [m_max, I], grown on demand
    uint64_t generation_ = 0;
};

// The split-K scratch shared by every prefill projection on a device (grow-only; see
// operators.cpp): a pointer to at least `bytes` (have = its size), and its current size.
void* linear_scratch(size_t bytes, int32_t device_id, size_t* have);
size_t linear_scratch_bytes(int32_t device_id);
// Number of times the device's scratch has been replaced (captured work that used the
// old buffer must be captured again).
uint64_t linear_scratch_generation(int32_t device_id);

// ---------------------------------------------------------------------------------
// Fused gate/up + SwiGLU (src/operators/fused_gate_up_activation_op.h:14-74). The
// fused weight is [up; gate] (src/layers/linear.cu:1923-1943).
// ---------------------------------------------------------------------------------
struct FusedGateUpActivationContext {
    ModelStage stage = ModelStage::Decode;
    int64_t m = 0, hidden = 0, intermediate = 0;
    DType dtype = DType::BFloat16;
};

struct FusedGateUpActivationState {
    bool available = false;
    std::string unavailable_reason;
};

class FusedGateUpActivationOp {
public:
    virtual ~FusedGateUpActivationOp() = default;
    virtual std::string impl_id() const = 0;
    virtual bool supports(const FusedGateUpActivationContext& ctx) const = 0;
    virtual FusedGateUpActivationState prepare(const FusedGateUpActivationContext& ctx, const Tensor& w_up_gate) = 0;
    virtual bool run(const FusedGateUpActivationContext& ctx, const Tensor& w_up_gate, const Tensor& input,
                     Tensor& output, hipStream_t stream) = 0;
};

class FusedGateUpActivationRegistry {
public:
    static FusedGateUpActivationRegistry& instance();
    FusedGateUpActivationOp* find_impl_by_id(const std::string& id) const;
    FusedGateUpActivationOp* default_impl(const FusedGateUpActivationContext& ctx) const;

private:
    FusedGateUpActivationRegistry();
    std::vector<std::unique_ptr<FusedGateUpActivationOp>> impls_;
};

// Resolve an implementation id for an operator query against the table (falls back to
// the registry default when the table has no record or the record's impl does not
// support the context: attention.cu:257-273).
std::string resolve_impl_id(const std::string& model_name, const std::string& hw_profile,
                            const std::string& table_path, const OperatorQuery& q, Json* impl_params = nullptr);

}  // namespace edge_fm
