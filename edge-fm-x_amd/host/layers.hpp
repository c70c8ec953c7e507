// Layer tier of the MI355X runtime: the reference's stand-alone layer classes
// (src/layers/*.h) that its Python bindings expose for per-layer use and testing
// (src/python/pybind_debug.cpp:486-1580). Each is built from an engine config (the
// model's config.json supplies the shapes), takes its weights from the WeightLoader's
// prefill stage (loading the config's checkpoint the first time a needed tensor is
// missing), resolves its operator impl from the operator table per stage exactly as the
// reference layer does, and runs the gfx950 kernels through the edgefm_hip C ABI.
//
// One checkpoint serves both stages (the engine loads no separate decode checkpoint), so
// decode-stage calls use the prefill-stage weights.
#pragma once

#include <array>
#include <string>
#include <unordered_map>
#include <vector>

#include "engine.hpp"
#include "operators.hpp"

namespace edge_fm {

// The prefill-stage weight map, after loading the engine config's checkpoint when none of
// `any_of` is registered yet (Qwen2.5-VL checkpoints: language model only, under text-model
// names; pybind_debug.cpp:62-106).
const std::unordered_map<std::string, Tensor>& layer_stage_weights(const EngineConfig& cfg,
                                                                   const std::vector<std::string>& any_of);

// ---------------------------------------------------------------------------------
// AttentionLayer (src/layers/attention.h:21-96, attention.cu:160-420)
// ---------------------------------------------------------------------------------
enum class RoPEMode { kNone, kRoPELlama, kMRoPE };

class AttentionLayer {
public:
    explicit AttentionLayer(const EngineConfig& engine_config, std::string layer_name = "");

    // q [qo_len, Hq, hd], k / v [kv_len, Hkv, hd], o [qo_len, Hq, hd]; strides in elements,
    // 0 = contiguous. RoPE-Llama on read unless the model uses M-RoPE (then none: M-RoPE is
    // applied beforehand by apply_mrope).
    void forward_prefill(const Tensor& q, const Tensor& k, const Tensor& v, Tensor& o, bool causal,
                         hipStream_t stream, uint32_t q_stride_n = 0, uint32_t q_stride_h = 0,
                         uint32_t kv_stride_n = 0, uint32_t kv_stride_h = 0, uint32_t k_stride_n = 0,
                         uint32_t k_stride_h = 0, bool k_already_prerotated = false,
                         uint32_t q_rope_pos_offset = 0, uint32_t k_rope_pos_offset = 0) const;
    // q [1, Hq, hd], k / v [kv_len or max_kv_len, Hkv, hd], o [1, Hq, hd]. With d_kv_len
    // (device, one uint32) the live length is read on the device and max_kv_len bounds it.
    void forward_decode(const Tensor& q, const Tensor& k, const Tensor& v, Tensor& o, hipStream_t stream,
                        uint32_t* d_kv_len = nullptr, uint32_t max_kv_len = 0) const;

    RoPEMode rope_mode() const { return rope_mode_; }
    std::string selected_impl_id(ModelStage stage) const;
    void reset_operator_impl_cache();

private:
    AttentionOpContext base_ctx() const;
    AttentionOp* resolve_impl(ModelStage stage) const;
    void check_tensor(const Tensor& t, const char* name) const;

    std::string model_name_, hw_profile_, table_path_, layer_name_;
    int32_t device_id_ = 0;
    DType dtype_ = DType::BFloat16;
    uint32_t num_qo_heads_ = 0, num_kv_heads_ = 0, head_dim_ = 0;
    float rope_theta_ = 1.0e6f, rope_scale_ = 1.0f;
    RoPEMode rope_mode_ = RoPEMode::kRoPELlama;
    mutable std::array<AttentionOp*, 2> selected_{{nullptr, nullptr}};
    mutable std::array<Json, 2> selected_params_{{Json::object(), Json::object()}};
};

// ---------------------------------------------------------------------------------
// RMSNormLayer (src/layers/layernorm.h, layernorm.cu:70-330)
// ---------------------------------------------------------------------------------
enum class NormWeightType { Input, PostAttention, Final };

class RMSNormLayer {
public:
    RMSNormLayer(uint32_t layer_id, NormWeightType weight_type, const EngineConfig& engine_config,
                 std::string layer_name = "");
    // model.layers.<id>.input_layernorm / post_attention_layernorm, or model.norm (Final or
    // layer_id UINT32_MAX); the weight must be [hidden_size].
    void load_weights(const std::unordered_map<std::string, Tensor>& prefill_weights);
    // output[b, :] = rmsnorm(input[b, :]) * w; input / output [batch, hidden]
    void forward_rmsnorm(const Tensor& input, Tensor& output, hipStream_t stream,
                         ModelStage stage = ModelStage::Prefill);
    // residual += inout; inout = rmsnorm(residual) * w (both [batch, hidden], in place)
    void forward_fused_add_rmsnorm(Tensor& inout, Tensor& residual, hipStream_t stream,
                                   ModelStage stage = ModelStage::Prefill);
    const std::string& layer_role() const { return role_; }
    std::string selected_impl_id(ModelStage stage) const;

private:
    NormOp* resolve_impl(const RMSNormOpContext& ctx, ModelStage stage);
    RMSNormOpContext make_ctx(const Tensor& a, const char* name) const;

    std::string model_name_, hw_profile_, table_path_, layer_name_, role_;
    int32_t device_id_ = 0;
    uint32_t layer_id_ = 0, hidden_ = 0;
    NormWeightType weight_type_ = NormWeightType::Input;
    float eps_ = 1e-6f;
    Tensor weight_;
    std::array<NormOp*, 2> selected_{{nullptr, nullptr}};
};

// ---------------------------------------------------------------------------------
// ActivationLayer (src/layers/activation.h, activation.cu:36-239): SiLU-and-mul over the
// last dimension, 2 * intermediate_size (or hidden_size) wide.
// ---------------------------------------------------------------------------------
class ActivationLayer {
public:
    explicit ActivationLayer(const EngineConfig& engine_config, std::string layer_name = "");
    // out = silu(x[..., :I]) * x[..., I:]   (flashinfer silu_and_mul layout)
    void forward_silu_and_mul(const Tensor& input, Tensor& output, hipStream_t stream,
                              ModelStage stage = ModelStage::Prefill);
    // out = silu(x[..., I:]) * x[..., :I]   (the fused [up; gate] projection's layout)
    void forward_silu_and_mul_up_gate(const Tensor& input, Tensor& output, hipStream_t stream,
                                      ModelStage stage = ModelStage::Prefill);
    std::string selected_impl_id(ModelStage stage) const;

private:
    void run(const Tensor& input, Tensor& output, hipStream_t stream, ModelStage stage, ActivationInputLayout layout);

    std::string model_name_, hw_profile_, table_path_, layer_name_;
    int32_t device_id_ = 0;
    uint32_t hidden_ = 0;
    std::array<ActivationOp*, 2> selected_{{nullptr, nullptr}};
};

// ---------------------------------------------------------------------------------
// SamplerLayer (src/layers/sampler.h, sampler.cu:121-298)
// ---------------------------------------------------------------------------------
class SamplerLayer {
public:
    explicit SamplerLayer(const EngineConfig& engine_config);
    // logits fp32 [batch, vocab] -> token_ids int32 [batch]. temperature < 1e-6: argmax
    // (lowest id among equal maxima); else row b draws from softmax(logits / T) restricted
    // to the top-p nucleus with Philox counter b and the configured seed (the same draws
    // on every call, as the reference's fixed seed and offset give).
    void forward_sampling(const Tensor& logits, Tensor& token_ids, hipStream_t stream);
    float temperature() const { return temperature_; }

private:
    int32_t device_id_ = 0;
    uint32_t vocab_ = 0;
    float temperature_ = 1.0f, top_p_ = 1.0f;
    uint64_t seed_ = 0;
};

// ---------------------------------------------------------------------------------
// EmbedHeadLayer (src/layers/embed_head.h, embed_head.cu:168-420)
// ---------------------------------------------------------------------------------
class EmbedHeadLayer {
public:
    explicit EmbedHeadLayer(const EngineConfig& engine_config, std::string layer_name = "");
    // model.embed_tokens.weight [vocab_size, hidden_size]
    void load_weights(const std::unordered_map<std::string, Tensor>& prefill_weights);
    // token_ids int32 [batch, seq] -> output [batch, seq, hidden] (ids outside the
    // vocabulary give zero rows)
    void forward_for_tokens(const Tensor& token_ids, Tensor& output, hipStream_t stream);
    // as forward_for_tokens, but ids in [embed_token_id, embed_token_id + rows) take rows of
    // `embeddings` [rows, hidden] (embed_token_id < 0: none do)
    void forward_for_embeddings(const Tensor& token_ids, const Tensor& embeddings, Tensor& output,
                                int32_t embed_token_id, hipStream_t stream);

private:
    void check_ids_out(const Tensor& token_ids, const Tensor& output) const;

    int32_t device_id_ = 0;
    uint32_t vocab_ = 0, hidden_ = 0;
    Tensor table_;
};

// ---------------------------------------------------------------------------------
// LMHeadLinearLayer (src/layers/linear.h, linear.cu:2229-2370): a LinearLayer whose weight
// is <prefix>.weight, model.<prefix>.weight or, tied, model.embed_tokens.weight.
// ---------------------------------------------------------------------------------
class LMHeadLinearLayer : public LinearLayer {
public:
    LMHeadLinearLayer(const std::string& layer_prefix, const EngineConfig& engine_config, uint32_t in_features,
                      uint32_t out_features, std::string layer_name = "");
    void load_weights(const std::unordered_map<std::string, Tensor>& prefill_weights);
    // Decode stage, no bias, bf16 input [1, hidden] and token_out int32 [1]: the greedy
    // token argmax(input . W^T) (lowest id among equal maxima) without materialising the
    // logits; returns false, having done nothing, for anything else.
    bool try_forward_top1(const Tensor& input, Tensor& token_out, hipStream_t stream,
                          ModelStage stage = ModelStage::Decode);

private:
    int32_t device_id_ = 0;
};

// Weights of the fused projections from a weight map (linear.cu:1640-1840, 1880-2045):
// [q; k; v] rows of <base>.{q,k,v}_proj.weight, with the biases concatenated (missing
// parts zero) when any is present; [up; gate] rows of <base>.{up,gate}_proj.weight.
// A map that already holds <base>.qkv_fused.weight / <base>.gate_up_fused.weight (and
// .bias) supplies those directly.
void load_fused_qkv_weights(FusedQKVLinearLayer& layer, const std::string& layer_prefix_base,
                            const std::unordered_map<std::string, Tensor>& weights, uint32_t q_out, uint32_t k_out,
                            uint32_t v_out, int32_t device_id);
void load_fused_gate_up_weights(FusedGateUpLinearLayer& layer, const std::string& layer_prefix_base,
                                const std::unordered_map<std::string, Tensor>& weights, int32_t device_id);

}  // namespace edge_fm
