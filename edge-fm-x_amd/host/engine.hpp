// Token-generation runtime of the MI355X EdgeFM engine: weight loading, engine
// configuration, fixed-prefix KV slots, the Qwen2.5 / Qwen2.5-VL model and the
// single-request generate loop with a HIP-graph-replayed decode step.
//
// Mirrors, in C++17 over HIP, the reference's src/engine (EngineConfig,
// engine_factory, StandardEngine, KVManager, Scheduler), src/models/qwen2_5 and
// src/utils/device/weight_loader.
#pragma once

#include <map>
#include <set>
#include <memory>
#include <mutex>
#include <string>
#include <unordered_map>
#include <vector>

#include "compact_vocab.hpp"
#include "core.hpp"
#include "json.hpp"
#include "operators.hpp"

namespace edge_fm {

// ---------------------------------------------------------------------------------
// WeightLoader (src/utils/device/weight_loader.h:20-120): per-stage name -> device
// tensor cache. Tensors come from safetensors files or are registered by the caller
// (device views, no copy).
// ---------------------------------------------------------------------------------
class WeightLoader {
public:
    static WeightLoader& instance();
    // Loads every tensor of the checkpoint at model_path (collect_safetensors_files) to
    // device memory. language_model_only (Qwen2.5-VL checkpoints,
    // src/engine/engine_factory.cpp:73-98): keep only the language model's tensors
    // (model., language_model., lm_head. names; the vision tower is not used) under
    // their text-model names (vl_language_model_name).
    void load_weights_from_file(const std::string& model_path, ModelStage stage, int32_t device_id,
                                bool language_model_only = false);
    void register_tensor(ModelStage stage, const std::string& name, const Tensor& t);
    const std::unordered_map<std::string, Tensor>& get(ModelStage stage);
    bool has_stage(ModelStage stage);
    void clear_stage(ModelStage stage);

private:
    std::mutex mu_;
    std::map<int, std::unordered_map<std::string, Tensor>> stages_;
};

// Parse one safetensors file into host-side descriptors (tests and tools use it).
struct SafetensorsEntry {
    std::string dtype;
    std::vector<int64_t> shape;
    size_t begin = 0, end = 0;
};
std::map<std::string, SafetensorsEntry> read_safetensors_header(const std::string& path, size_t* data_offset);

// The checkpoint files of a model path (src/engine/engine_factory.cpp:27-49): the path
// itself when it is a file; else <dir>/model.safetensors when present; else every
// <dir>/model-*-of-*.safetensors shard in name order. None: ConfigurationError.
std::vector<std::string> collect_safetensors_files(const std::string& model_path);

// Text-model name of a Qwen2.5-VL checkpoint tensor: model.language_model.X and
// model.model.X -> model.X, language_model.X -> X; names of the vision tower (anything
// not under model., language_model. or lm_head.) -> "" (not loaded).
std::string vl_language_model_name(const std::string& name);

// ---------------------------------------------------------------------------------
// EngineConfig (src/engine/engine.h:29-89): engine_default.json merged with the user
// JSON (src/engine/engine.cpp:207-212).
// ---------------------------------------------------------------------------------
struct KVSlotConfig {
    int32_t request_id = 0;
    std::vector<int32_t> prefix_token_ids;
    int32_t max_tokens = 4096;
};

class EngineConfig {
public:
    explicit EngineConfig(const std::string& config_path);
    static std::string default_config_dir();

    const Json& json() const { return json_; }
    std::string model_name() const;
    int32_t device_id() const;
    std::string hw_profile() const;
    bool use_graph() const;
    bool lm_head_top1() const;
    // runtime.debug_logits: every generated token's fp32 logits are kept on the device
    // (logits path instead of the fused LM-head top-1) and returned by
    // EdgeFM::last_logits() (test and debugging aid; off by default)
    bool debug_logits() const;
    // Whether the one-launch input norm + QKV + attention partials impl
    // (hip_gfx950_decode_fused_qkv_attention) may run when an operator-table record
    // selects it (runtime.decode_fused_qkv_attention, default on;
    // EDGE_FM_DECODE_FUSED_QKV_ATTENTION = 1 / 0 overrides the config).
    bool decode_fused_qkv_attention() const;
    std::string operator_table_path() const;
    std::string prefill_model_path() const;
    std::vector<KVSlotConfig> kv_slots() const;
    int32_t max_new_tokens() const;
    float temperature() const;
    float top_p() const;
    uint64_t seed() const;
    std::vector<int32_t> stop_token_ids() const;
    const Json& model_config() const { return model_json_; }
    std::vector<int32_t> eos_token_ids() const;
    // "compact_vocab" object of the merged config, or an empty object.
    Json compact_vocab() const;
    // Directory of the user config file (relative paths in it resolve against it).
    const std::string& config_dir() const { return base_dir_; }

private:
    Json json_;
    Json model_json_;
    std::string base_dir_;
};

// Hyper-parameters read from the model's config.json (HF Qwen2 / Qwen2.5-VL format).
struct ModelConfig {
    int32_t hidden = 0, inter = 0, layers = 0, heads = 0, kv_heads = 0, head_dim = 0;
    int64_t vocab = 0;
    float eps = 1e-6f, theta = 1.0e6f;
    bool tied = true;
    bool mrope = false;
    int32_t mrope_section[3] = {0, 0, 0};
    static ModelConfig from_json(const Json& j);
    int32_t q_dim() const { return heads * head_dim; }
    int32_t kv_dim() const { return kv_heads * head_dim; }
};

// ---------------------------------------------------------------------------------
// Decode plan: the impls one decode layer runs, resolved from the operator table at
// stage "decode" like the reference's AttentionLayer / LinearLayer / FusedGateUpLinearLayer
// (src/layers/attention.cu:211-276, src/operators/linear_impl.cu:866-915):
//   attention  AttentionOp for (op_kind attention, op_name attention, stage decode,
//              shape_sig "num_qo_heads=..|num_kv_heads=..|head_dim=.."); a record naming an
//              impl that does not support the shape falls back to the registry default
//              (fused launch, split partials, generic attention, in that order)
//   o_proj     LinearLayer impl of model.layers.<l>.self_attn.o_proj at (decode, m = 1)
//   gate_up    FusedGateUpActivationOp at (decode, op_name model.layers.<l>.mlp), run with
//              the post-attention norm as its prologue; "" when no impl supports the
//              shape (norm, gate/up linear, activation as three launches)
//   down       LinearLayer impl of model.layers.<l>.mlp.down_proj at (decode, m = 1)
// An attention impl that leaves split partials needs the merge-in-prologue o_proj
// (hip_gfx950_decode_merge_o_proj); the fused launch with any other o_proj is a
// ConfigurationError, the split impl then runs with its in-kernel merge.
// ---------------------------------------------------------------------------------
struct DecodeLayerPlan {
    std::string attention, o_proj, gate_up, down;
    bool partials_to_o_proj = false;   // attention leaves split partials; o_proj merges them
};

class LinearLayer;
// Resolve one decode layer for caches of up to max_kv_len rows. allow_fused_front: the
// engine config permits the fused norm + QKV + attention launch.
DecodeLayerPlan resolve_decode_layer(const EngineConfig& cfg, const ModelConfig& m, int32_t layer,
                                     uint32_t max_kv_len, bool allow_fused_front, LinearLayer& o_proj,
                                     LinearLayer& down);
// The plan of every layer of the model an engine config describes, with no device work
// (the engine resolves the same plan when it reserves its decode scratch).
std::vector<DecodeLayerPlan> plan_decode(const std::string& engine_config_path, uint32_t max_kv_len);

// ---------------------------------------------------------------------------------
// KVManager (src/engine/tasks/token_generation/kv_manager.h:58-106): one contiguous
// buffer per request slot, laid out [layer][K | V][max_tokens][Hkv * hd] bf16.
// ---------------------------------------------------------------------------------
struct KVSlot {
    KVSlotConfig cfg;
    Tensor buffer;
    int32_t prefix_size = 0;
    bool prefix_ready = false;
};

struct KVSlotStatus {
    int32_t request_id = 0;
    std::vector<int32_t> prefix_token_ids;
    size_t prefix_size = 0;
    int32_t max_tokens = 0;
    size_t allocated_size = 0;   // bytes over all layers
};
struct KVManagerStatus {
    std::vector<KVSlotStatus> slots;
    Device device = Device::GPU;
    int32_t device_id = 0;
};

class KVManager {
public:
    KVManager(const std::vector<KVSlotConfig>& slots, const ModelConfig& m, int32_t device_id);
    // The slots of the config's kvcache.requests (prefix ids remapped through the config's
    // compact vocabulary, kv_manager.cpp:45-190).
    explicit KVManager(const EngineConfig& engine_config);
    KVSlot& slot(int32_t request_id);
    bool is_request_valid(int32_t request_id) const;
    void* k_cache(int32_t request_id, int layer);
    void* v_cache(int32_t request_id, int layer);
    std::vector<int32_t> request_ids() const;
    // Per layer: the start of the layer's [K | V] block, and that start advanced past the
    // fixed prefix's K rows (the first row a request writes), kv_manager.cpp:248-262.
    std::vector<void*> get_read_kvcache(int32_t request_id) const;
    std::vector<void*> get_write_kvcache(int32_t request_id) const;
    KVManagerStatus get_status() const;

private:
    const KVSlot& find(int32_t request_id) const;
    ModelConfig m_;
    int32_t device_id_ = 0;
    std::vector<KVSlot> slots_;
};

// Rows of `parts` stacked into one new bf16 device tensor (2-D parts share their column
// count), copied on `stream`.
Tensor concat_rows(const std::vector<const Tensor*>& parts, int32_t device_id, hipStream_t stream);

// ---------------------------------------------------------------------------------
// Qwen2.5 model (src/models/qwen2_5/qwen2_5.cpp:84-980)
// ---------------------------------------------------------------------------------
class Qwen2_5 {
public:
    Qwen2_5(const EngineConfig& cfg, const ModelConfig& m, const std::unordered_map<std::string, Tensor>& weights,
            int32_t device_id);

    const ModelConfig& config() const { return m_; }

    // Prefill S tokens into cache rows [base, base + S) of (k_caches, v_caches).
    // ids: device int32 [S]; embeddings (optional) device bf16 [n_custom, H];
    // position_ids (M-RoPE) device int32 [3, S]. Writes the greedy token of the last
    // row into token_out (device int32[1]) or, if logits != nullptr, fp32 logits.
    void prefill(int32_t S, int32_t base, const int32_t* ids, const Tensor* embeddings, int32_t embed_token_id,
                 const int32_t* position_ids, void** k_caches, void** v_caches, int32_t* token_out, float* logits,
                 hipStream_t stream);

    // One decode step for the token in token_buf (device int32[1]) at cache length
    // *d_kv_len (device). Graph-capturable: no allocation, no host reads.
    void decode_step(int32_t* token_buf, const uint32_t* d_kv_len, uint32_t max_kv_len, const int32_t* d_pos3,
                     void** k_caches, void** v_caches, float* logits, hipStream_t stream);

    // Allocate the decode scratch for caches of up to max_kv_len rows (must run before
    // a decode step is captured into a graph: capture cannot allocate).
    void reserve_decode(uint32_t max_kv_len);

    // Changes whenever a buffer that prefill reads or writes is replaced (its grow-only
    // scratch, the MLP intermediate, the shared split-K scratch): a captured prefill is
    // valid only while this is unchanged.
    uint64_t prefill_buffers_epoch() const;

    // Whether decode steps run efm_decode_norm_qkv_attention (input norm + QKV +
    // attention partials in one launch per layer) in every layer.
    bool uses_fused_front(uint32_t max_kv_len) const;
    // The decode plan for caches of max_kv_len rows (resolved by reserve_decode).
    const std::vector<DecodeLayerPlan>& decode_plan(uint32_t max_kv_len) const;
    // Throws DeviceError if a fused QKV + attention launch since the last
    // check could not exchange its vectors in time (synchronises the stream).
    void check_decode_status(hipStream_t stream);

private:
    struct Layer {
        Tensor qkv_w, qkv_b, o_w, gu_w, down_w, in_norm, post_norm;
        // LinearLayers over the tensors above, under the reference's prefixes
        // (self_attn [fused_qkv], self_attn.o_proj, mlp [fused_gate_up], mlp.down_proj)
        std::unique_ptr<LinearLayer> qkv, o_proj, gate_up, down;
    };
    const EngineConfig& cfg_;
    ModelConfig m_;
    int32_t device_id_;
    std::string model_name_, hw_profile_, table_path_;
    Tensor embed_, lm_head_, final_norm_;
    std::vector<Layer> layers_;
    // operator instances resolved from the implementation table
    AttentionOp* attn_ = nullptr;
    NormOp* norm_ = nullptr;
    FusedGateUpActivationOp* swiglu_ = nullptr;
    ActivationOp* act_ = nullptr;
    std::unique_ptr<PrefillMlpSourceOp> mlp_source_;
    // decode plans per cache length (reserve_decode)
    std::map<uint32_t, std::vector<DecodeLayerPlan>> plans_;
    Tensor dec_gu_;   // [1, 2 I] gate/up output of the layered decode MLP
    // decode scratch
    Tensor dec_h_, dec_res_[2], dec_q_, dec_attn_, dec_a_, dec_mid_, dec_kvtmp_, dec_one_, top1_ws_;
    Tensor attn_ws_;
    bool fused_front_enabled_ = false;
    Tensor front_sync_ws_;
    // prefill scratch (grow-only)
    int32_t pf_cap_ = 0;
    uint64_t pf_epoch_ = 0;
    Tensor pf_hidden_, pf_res_, pf_norm_, pf_qkv_, pf_attn_, pf_mid_;

    const Tensor& w(const std::unordered_map<std::string, Tensor>& ws, const std::string& name) const;
    void ensure_prefill_capacity(int32_t S);
    efm_attention_ctx decode_ctx() const;
    efm_attention_ctx decode_attn_ctx_rotated() const;
    AttentionOpContext attn_ctx() const;
};

// ---------------------------------------------------------------------------------
// StandardEngine + EdgeFM facade (include/edge-fm/edge-fm.h:10-111)
// ---------------------------------------------------------------------------------
class StandardEngine {
public:
    explicit StandardEngine(const std::string& config_path);
    ~StandardEngine();
    Response generate(const Request& request);
    std::unordered_map<std::string, double> last_generate_metrics() const { return metrics_; }
    const ModelConfig& model_config() const { return model_->config(); }
    const EngineConfig& engine_config() const { return cfg_; }
    const CompactVocab& compact_vocab() const { return compact_vocab_; }
    void warmup();
    // fp32 logits of every token of the last generate() call ([rows, vocab], row-major),
    // with runtime.debug_logits set; ConfigurationError otherwise
    std::vector<float> last_logits(int32_t* rows, int32_t* vocab) const;

private:
    EngineConfig cfg_;
    CompactVocab compact_vocab_;
    int32_t device_id_;
    hipStream_t stream_ = nullptr;
    std::unique_ptr<Qwen2_5> model_;
    std::unique_ptr<KVManager> kv_;
    std::unordered_map<std::string, double> metrics_;
    // device decode state: [0] d_kv_len, [1] d_step, [2] token, [3..5] M-RoPE position
    Tensor state_;
    Tensor response_dev_;
    Tensor ids_dev_;
    Tensor logits_;
    Tensor logits_hist_;     // runtime.debug_logits: [response slots, vocab] fp32
    int32_t last_n_gen_ = 0;
    Tensor sample_ws_;
    // One decode step, and kGraphSteps consecutive steps in one graph (fewer graph launches:
    // each costs a few us of command-processor time between the steps it separates).
    static constexpr int32_t kGraphSteps = 8;
    struct GraphEntry {
        hipGraph_t graph = nullptr;
        hipGraphExec_t exec = nullptr;
        hipGraph_t graph_n = nullptr;
        hipGraphExec_t exec_n = nullptr;
    };
    // per (request slot, row bound): a decode step reads cache rows below the bound that
    // its launches were built for, so graphs are captured per 128-row bucket of the
    // lengths their steps reach (decode_row_bound)
    std::map<std::pair<int32_t, uint32_t>, GraphEntry> graphs_;
    void drop_graphs();
    // Row bound of decode steps whose longest attended length is `rows`: the 128-row
    // bucket holding it (the split plan's unit), at most the slot's capacity. Split b
    // requests rows [128 b, 128 b + 128) below the bound before the device-side length is
    // read, so a bound near the length keeps those reads to live rows.
    static constexpr uint32_t kDecodeBoundRows = 128;
    static uint32_t decode_row_bound(uint32_t rows, uint32_t capacity);

    // Prefill graphs (standard_engine.cpp:568-800): one per (request slot, prefilled rows,
    // cache base row, custom embedding rows, embed_token_id), captured the second time a
    // key is prefilled (the first, eager, run sizes every buffer the capture then reads)
    // and replayed after that. The request's ids, custom embeddings and M-RoPE positions
    // are staged into the persistent buffers below first, so a replay reads this call's
    // inputs. A graph is dropped when a buffer it uses has been replaced since capture.
    using PrefillKey = std::tuple<int32_t, int32_t, int32_t, int64_t, int32_t>;
    struct PrefillGraph {
        hipGraph_t graph = nullptr;
        hipGraphExec_t exec = nullptr;
        uint64_t epoch = 0;
    };
    static constexpr size_t kMaxPrefillGraphs = 32;
    std::map<PrefillKey, PrefillGraph> pf_graphs_;
    std::set<PrefillKey> pf_seen_;
    Tensor pf_emb_dev_, pf_pos_dev_;
    uint64_t pf_input_epoch_ = 0;
    uint64_t prefill_epoch() const;
    void drop_prefill_graphs();

    // stage_events: StageEvents of the eager loop's per-step timing, or null (captured)
    void run_decode_step(int32_t request_id, void* stage_events, uint32_t row_bound);
    void sample_logits(uint32_t step_index);
    std::vector<void*> caches(int32_t request_id, bool k);
};

class EdgeFM {
public:
    explicit EdgeFM(const std::string& config_path);
    Response generate(const Request& request) const;
    std::unordered_map<std::string, double> last_generate_metrics() const;
    std::vector<float> last_logits(int32_t* rows, int32_t* vocab) const;
    const StandardEngine& engine() const { return *engine_; }

private:
    std::unique_ptr<StandardEngine> engine_;
};

}  // namespace edge_fm
