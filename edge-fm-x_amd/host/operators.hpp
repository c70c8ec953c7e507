// Operator layer of the MI355X runtime: the reference's operator interfaces
// (src/operators/*.h, src/layers/linear.h:110-153), their registries and the
// operator implementation table, with gfx950 implementations that call the
// edgefm_hip C ABI.
#pragma once

#include <memory>
#include <mutex>
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
};

efm_attention_ctx to_c_ctx(const AttentionOpContext& c);

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
// Linear (LinearLayer::LinearImpl, src/layers/linear.h:110-153; registry
// src/operators/linear_registry.h:9-24). layer_role is one of fused_qkv,
// attention_output, fused_gate_up, mlp_down, lm_head.
// ---------------------------------------------------------------------------------
struct LinearShape {
    int64_t m = 0;
    DType input = DType::BFloat16, weight = DType::BFloat16, output = DType::BFloat16;
    int64_t in_features = 0, out_features = 0;
};

struct LinearOpContext {
    std::string layer_prefix, layer_role;
    ModelStage stage = ModelStage::Decode;
    LinearShape shape;
    bool has_bias = false;
    Json impl_params = Json::object();
};

std::string linear_shape_sig(const LinearShape& s);

class LinearImpl {
public:
    virtual ~LinearImpl() = default;
    virtual std::string impl_id() const = 0;
    virtual bool supports(const LinearOpContext& ctx) const = 0;
    virtual void forward(const LinearOpContext& ctx, const Tensor& weight, const Tensor* bias, const Tensor& input,
                         Tensor& output, hipStream_t stream) = 0;
};

class LinearOpRegistry {
public:
    static LinearOpRegistry& instance();
    LinearImpl* find_impl_by_id(const std::string& id) const;
    LinearImpl* default_impl(const LinearOpContext& ctx) const;

private:
    LinearOpRegistry();
    std::vector<std::unique_ptr<LinearImpl>> impls_;
};

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
