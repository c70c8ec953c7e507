// Python bindings of the layer tier (the reference's per-layer bindings,
// src/python/pybind_debug.cpp:486-1580): the same class names, constructor arguments,
// method names, argument names and defaults. Streams are passed as integers (0 = the
// null stream); stages as "Prefill" / "Decode". Layers built from a config path take
// their weights from the WeightLoader's prefill stage, loading the config's checkpoint
// the first time a tensor they need is missing.
#include <pybind11/pybind11.h>
#include <pybind11/stl.h>

#include "layers.hpp"

namespace py = pybind11;

namespace edge_fm {

namespace {

hipStream_t as_stream(uintptr_t s) { return reinterpret_cast<hipStream_t>(s); }
ModelStage as_stage(const std::string& s) { return s == "Decode" ? ModelStage::Decode : ModelStage::Prefill; }

const Tensor& need(const std::unordered_map<std::string, Tensor>& w, const std::string& name) {
    auto it = w.find(name);
    if (it == w.end()) throw ConfigurationError("weight not found: " + name);
    return it->second;
}

const Tensor* maybe(const std::unordered_map<std::string, Tensor>& w, const std::string& name) {
    auto it = w.find(name);
    return it == w.end() ? nullptr : &it->second;
}

std::string impl_info(LinearLayer& self, ModelStage stage, int32_t m) {
    Json j = Json::object();
    j["layer_prefix"] = self.layer_prefix();
    j["layer_role"] = self.layer_role();
    j["stage"] = stage == ModelStage::Decode ? "decode" : "prefill";
    j["m"] = (int64_t)m;
    j["selected_impl_id"] = self.selected_impl_id(stage, m);
    LinearLayer::LinearShapeSignature sig;
    sig.m = m;
    sig.in_features = self.in_features();
    sig.out_features = self.out_features();
    j["shape_sig"] = sig.to_string();
    return j.dump();
}

std::string weight_info(LinearLayer& self, ModelStage stage) {
    Json j = Json::object();
    const Tensor* w = self.weight_tensor(stage);
    const Tensor* b = self.bias_tensor(stage);
    Json shape = Json::array();
    if (w)
        for (int64_t d : w->shape()) shape.push_back(d);
    j["weight_shape"] = shape;
    j["weight_dtype"] = w ? dtype_name(w->dtype()) : "";
    j["has_bias"] = b != nullptr;
    return j.dump();
}

}  // namespace

void bind_layers(py::module_& m) {
    py::class_<AttentionLayer>(m, "AttentionLayer")
        .def(py::init([](const std::string& config_path) {
                 return std::make_unique<AttentionLayer>(EngineConfig(config_path));
             }),
             py::arg("config_path"))
        .def("forward_prefill",
             [](AttentionLayer& self, const Tensor& q, const Tensor& k, const Tensor& v, Tensor& o, bool causal,
                uintptr_t stream, uint32_t q_stride_n, uint32_t q_stride_h, uint32_t kv_stride_n,
                uint32_t kv_stride_h, uint32_t k_stride_n, uint32_t k_stride_h) {
                 self.forward_prefill(q, k, v, o, causal, as_stream(stream), q_stride_n, q_stride_h, kv_stride_n,
                                      kv_stride_h, k_stride_n, k_stride_h);
             },
             py::arg("q"), py::arg("k"), py::arg("v"), py::arg("o"), py::arg("causal") = true, py::arg("stream") = 0,
             py::arg("q_stride_n") = 0, py::arg("q_stride_h") = 0, py::arg("kv_stride_n") = 0,
             py::arg("kv_stride_h") = 0, py::arg("k_stride_n") = 0, py::arg("k_stride_h") = 0)
        .def("forward_decode",
             [](AttentionLayer& self, const Tensor& q, const Tensor& k, const Tensor& v, Tensor& o, uintptr_t stream,
                uint32_t max_kv_len, const Tensor* d_kv_len) {
                 uint32_t* d = d_kv_len ? static_cast<uint32_t*>(d_kv_len->data_ptr()) : nullptr;
                 self.forward_decode(q, k, v, o, as_stream(stream), d, max_kv_len);
             },
             py::arg("q"), py::arg("k"), py::arg("v"), py::arg("o"), py::arg("stream") = 0, py::arg("max_kv_len") = 0,
             py::arg("d_kv_len") = static_cast<const Tensor*>(nullptr))
        .def("selected_impl_id", [](const AttentionLayer& self, const std::string& stage) {
            return self.selected_impl_id(as_stage(stage));
        }, py::arg("stage") = "Prefill");

    py::class_<RMSNormLayer>(m, "RMSNormLayer")
        .def(py::init([](uint32_t layer_id, const std::string& config_path, const std::string& weight_type) {
                 EngineConfig cfg(config_path);
                 NormWeightType wt = NormWeightType::Input;
                 std::string name = "model.layers." + std::to_string(layer_id) + ".input_layernorm.weight";
                 if (weight_type == "post_attention") {
                     wt = NormWeightType::PostAttention;
                     name = "model.layers." + std::to_string(layer_id) + ".post_attention_layernorm.weight";
                 } else if (weight_type == "final") {
                     wt = NormWeightType::Final;
                     name = "model.norm.weight";
                 }
                 auto layer = std::make_unique<RMSNormLayer>(layer_id, wt, cfg);
                 layer->load_weights(layer_stage_weights(cfg, {name}));
                 return layer;
             }),
             py::arg("layer_id"), py::arg("config_path"), py::arg("weight_type") = "input")
        .def("forward_rmsnorm",
             [](RMSNormLayer& self, const Tensor& input, Tensor& output, uintptr_t stream) {
                 self.forward_rmsnorm(input, output, as_stream(stream));
             },
             py::arg("input"), py::arg("output"), py::arg("stream") = 0)
        .def("forward_fused_add_rmsnorm",
             [](RMSNormLayer& self, Tensor& inout, Tensor& residual, uintptr_t stream) {
                 self.forward_fused_add_rmsnorm(inout, residual, as_stream(stream));
             },
             py::arg("inout"), py::arg("residual"), py::arg("stream") = 0)
        .def("layer_role", &RMSNormLayer::layer_role);

    py::class_<ActivationLayer>(m, "ActivationLayer")
        .def(py::init([](const std::string& config_path) {
                 return std::make_unique<ActivationLayer>(EngineConfig(config_path));
             }),
             py::arg("config_path"))
        .def("forward_silu_and_mul",
             [](ActivationLayer& self, const Tensor& input, Tensor& output, uintptr_t stream, const std::string& stage) {
                 self.forward_silu_and_mul(input, output, as_stream(stream), as_stage(stage));
             },
             py::arg("input"), py::arg("output"), py::arg("stream") = 0, py::arg("stage") = "Prefill")
        .def("forward_silu_and_mul_up_gate",
             [](ActivationLayer& self, const Tensor& input, Tensor& output, uintptr_t stream, const std::string& stage) {
                 self.forward_silu_and_mul_up_gate(input, output, as_stream(stream), as_stage(stage));
             },
             py::arg("input"), py::arg("output"), py::arg("stream") = 0, py::arg("stage") = "Prefill");

    py::class_<SamplerLayer>(m, "SamplerLayer")
        .def(py::init([](const std::string& config_path) {
                 return std::make_unique<SamplerLayer>(EngineConfig(config_path));
             }),
             py::arg("config_path"))
        .def("forward",
             [](SamplerLayer& self, const Tensor& logits, Tensor& token_ids, uintptr_t stream) {
                 self.forward_sampling(logits, token_ids, as_stream(stream));
             },
             py::arg("logits"), py::arg("token_ids"), py::arg("stream") = 0);

    py::class_<LinearLayer>(m, "LinearLayer")
        .def(py::init([](const std::string& layer_prefix, const std::string& config_path, uint32_t in_features,
                         uint32_t out_features) {
                 EngineConfig cfg(config_path);
                 const auto& w = layer_stage_weights(cfg, {layer_prefix + ".weight"});
                 auto layer = std::make_unique<LinearLayer>(layer_prefix, cfg, in_features, out_features);
                 layer->load_weights(need(w, layer_prefix + ".weight"), maybe(w, layer_prefix + ".bias"));
                 return layer;
             }),
             py::arg("layer_prefix"), py::arg("config_path"), py::arg("in_features"), py::arg("out_features"))
        .def("forward_fp16_bf16",
             [](LinearLayer& self, const Tensor& input, Tensor& output, uintptr_t stream, const std::string& stage) {
                 self.forward_fp16_bf16(input, output, as_stream(stream), as_stage(stage));
             },
             py::arg("input"), py::arg("output"), py::arg("stream") = 0, py::arg("stage") = "Prefill")
        .def("debug_cached_impl_info",
             [](LinearLayer& self, const std::string& stage, int32_t m) { return impl_info(self, as_stage(stage), m); },
             py::arg("stage") = "Decode", py::arg("m") = 1)
        .def("debug_weight_tensor_info",
             [](LinearLayer& self, const std::string& stage) { return weight_info(self, as_stage(stage)); },
             py::arg("stage") = "Prefill");

    py::class_<FusedQKVLinearLayer, LinearLayer>(m, "FusedQKVLinearLayer")
        .def(py::init([](const std::string& base, const std::string& config_path, uint32_t in_features,
                         uint32_t q_out, uint32_t k_out, uint32_t v_out) {
                 EngineConfig cfg(config_path);
                 const auto& w = layer_stage_weights(cfg, {base + ".q_proj.weight", base + ".qkv_fused.weight"});
                 auto layer = std::make_unique<FusedQKVLinearLayer>(base, cfg, in_features, q_out, k_out, v_out);
                 load_fused_qkv_weights(*layer, base, w, q_out, k_out, v_out, cfg.device_id());
                 return layer;
             }),
             py::arg("layer_prefix_base"), py::arg("config_path"), py::arg("in_features"), py::arg("q_out_features"),
             py::arg("k_out_features"), py::arg("v_out_features"));

    py::class_<FusedGateUpLinearLayer, LinearLayer>(m, "FusedGateUpLinearLayer")
        .def(py::init([](const std::string& base, const std::string& config_path, uint32_t in_features,
                         uint32_t gate_out, uint32_t up_out) {
                 EngineConfig cfg(config_path);
                 const auto& w = layer_stage_weights(cfg, {base + ".up_proj.weight", base + ".gate_up_fused.weight"});
                 auto layer = std::make_unique<FusedGateUpLinearLayer>(base, cfg, in_features, gate_out, up_out);
                 load_fused_gate_up_weights(*layer, base, w, cfg.device_id());
                 return layer;
             }),
             py::arg("layer_prefix_base"), py::arg("config_path"), py::arg("in_features"),
             py::arg("gate_out_features"), py::arg("up_out_features"))
        .def("try_forward_decode_swiglu_fused",
             [](FusedGateUpLinearLayer& self, const Tensor& input, Tensor& output, uintptr_t stream) {
                 return self.try_forward_decode_swiglu_fused(input, output, as_stream(stream));
             },
             py::arg("input"), py::arg("output"), py::arg("stream") = 0)
        .def("try_forward_prefill_swiglu_fused",
             [](FusedGateUpLinearLayer& self, const Tensor& input, Tensor& output, uintptr_t stream) {
                 return self.try_forward_prefill_swiglu_fused(input, output, as_stream(stream));
             },
             py::arg("input"), py::arg("output"), py::arg("stream") = 0);

    py::class_<LMHeadLinearLayer, LinearLayer>(m, "LMHeadLinearLayer")
        .def(py::init([](const std::string& config_path, uint32_t in_features, uint32_t out_features,
                         const std::string& layer_prefix) {
                 EngineConfig cfg(config_path);
                 const auto& w = layer_stage_weights(
                     cfg, {layer_prefix + ".weight", "model." + layer_prefix + ".weight", "model.embed_tokens.weight"});
                 auto layer = std::make_unique<LMHeadLinearLayer>(layer_prefix, cfg, in_features, out_features);
                 layer->load_weights(w);
                 return layer;
             }),
             py::arg("config_path"), py::arg("in_features"), py::arg("out_features"),
             py::arg("layer_prefix") = "lm_head")
        .def("try_forward_top1",
             [](LMHeadLinearLayer& self, const Tensor& input, Tensor& token_out, uintptr_t stream,
                const std::string& stage) {
                 return self.try_forward_top1(input, token_out, as_stream(stream), as_stage(stage));
             },
             py::arg("input"), py::arg("token_out"), py::arg("stream") = 0, py::arg("stage") = "Decode");

    py::class_<EmbedHeadLayer>(m, "EmbedHeadLayer")
        .def(py::init([](const std::string& config_path) {
                 EngineConfig cfg(config_path);
                 auto layer = std::make_unique<EmbedHeadLayer>(cfg);
                 layer->load_weights(layer_stage_weights(cfg, {"model.embed_tokens.weight"}));
                 return layer;
             }),
             py::arg("config_path"))
        .def("forward_for_tokens",
             [](EmbedHeadLayer& self, const Tensor& token_ids, Tensor& output, uintptr_t stream) {
                 self.forward_for_tokens(token_ids, output, as_stream(stream));
             },
             py::arg("token_ids"), py::arg("output"), py::arg("stream") = 0)
        .def("forward_for_embeddings",
             [](EmbedHeadLayer& self, const Tensor& token_ids, const Tensor& embeddings, Tensor& output,
                int32_t embed_token_id, uintptr_t stream) {
                 self.forward_for_embeddings(token_ids, embeddings, output, embed_token_id, as_stream(stream));
             },
             py::arg("token_ids"), py::arg("embeddings"), py::arg("output"), py::arg("embed_token_id") = -1,
             py::arg("stream") = 0);

    py::class_<KVSlotStatus>(m, "KVSlotStatus")
        .def_readonly("request_id", &KVSlotStatus::request_id)
        .def_readonly("prefix_token_ids", &KVSlotStatus::prefix_token_ids)
        .def_readonly("prefix_size", &KVSlotStatus::prefix_size)
        .def_readonly("max_tokens", &KVSlotStatus::max_tokens)
        .def_readonly("allocated_size", &KVSlotStatus::allocated_size);
    py::class_<KVManagerStatus>(m, "KVManagerStatus")
        .def_readonly("slots", &KVManagerStatus::slots)
        .def_readonly("device", &KVManagerStatus::device)
        .def_readonly("device_id", &KVManagerStatus::device_id);
    py::class_<KVManager>(m, "KVManager")
        .def(py::init([](const std::string& config_path) {
                 return std::make_unique<KVManager>(EngineConfig(config_path));
             }),
             py::arg("config_path"))
        .def("get_read_kvcache",
             [](const KVManager& self, int32_t request_id) {
                 std::vector<uintptr_t> out;
                 for (void* p : self.get_read_kvcache(request_id)) out.push_back(reinterpret_cast<uintptr_t>(p));
                 return out;
             },
             py::arg("request_id"))
        .def("get_write_kvcache",
             [](const KVManager& self, int32_t request_id) {
                 std::vector<uintptr_t> out;
                 for (void* p : self.get_write_kvcache(request_id)) out.push_back(reinterpret_cast<uintptr_t>(p));
                 return out;
             },
             py::arg("request_id"))
        .def("get_status", &KVManager::get_status)
        .def("is_request_valid", &KVManager::is_request_valid, py::arg("request_id"));
}

}  // namespace edge_fm
