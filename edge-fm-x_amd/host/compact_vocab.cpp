// Compact-vocabulary id mapping (src/engine/tasks/token_generation/compact_vocab.cpp).
#include "compact_vocab.hpp"

#include <filesystem>

#include "engine.hpp"
#include "json.hpp"

namespace fs = std::filesystem;

namespace edge_fm {

namespace {

constexpr const char* kCompactVocabFormat = "edgefm.compact_vocab.v1";

Json load_mapping(const std::string& path) {
    if (!fs::exists(path)) throw ConfigurationError("Cannot open compact_vocab mapping file: " + path);
    try {
        return Json::parse_file(path);
    } catch (const std::exception& e) {
        throw ConfigurationError("Failed to parse compact_vocab mapping file " + path + ": " + e.what());
    }
}

int32_t required_int(const Json& j, const std::string& key) {
    check<ConfigurationError>(j.contains(key) && j.at(key).is_integer(),
                              "compact_vocab mapping requires integer field: " + key);
    return (int32_t)j.at(key).as_int();
}

std::vector<int32_t> required_int_array(const Json& j, const std::string& key) {
    check<ConfigurationError>(j.contains(key) && j.at(key).is_array(),
                              "compact_vocab mapping requires integer array field: " + key);
    std::vector<int32_t> out;
    out.reserve(j.at(key).size());
    for (const Json& v : j.at(key).as_array()) {
        check<ConfigurationError>(v.is_integer(), "compact_vocab mapping field " + key + " must contain only integers");
        out.push_back((int32_t)v.as_int());
    }
    return out;
}

// Relative mapping paths resolve against the user config's directory (:54-63).
std::string resolve_mapping_path(const EngineConfig& config, const std::string& raw) {
    check<ConfigurationError>(!raw.empty(), "compact_vocab.enabled=true requires compact_vocab.mapping_path");
    fs::path p(raw);
    if (p.is_relative()) p = fs::path(config.config_dir()) / p;
    return p.lexically_normal().string();
}

// v1 runs a pre-pruned checkpoint: its vocab_size must equal the compact size (:65-84).
// Qwen2.5-VL configs that keep vocab_size under text_config are read from there.
void validate_model_vocab_size(const EngineConfig& config, int32_t compact) {
    const Json& mc = config.model_config();
    const Json* src = &mc;
    if (!mc.contains("vocab_size") && mc.contains("text_config")) src = &mc.at("text_config");
    check<ConfigurationError>(src->contains("vocab_size") && src->at("vocab_size").is_integer(),
                              "compact_vocab requires prefill_model.config.json to define integer vocab_size");
    const int64_t v = src->at("vocab_size").as_int();
    check<ConfigurationError>(v == compact,
                              "compact_vocab v1 expects pre-pruned checkpoint vocab_size == compact_vocab_size. "
                              "prefill_model vocab_size=" + std::to_string(v) +
                                  ", compact_vocab_size=" + std::to_string(compact));
}

std::string ids_context(const std::string& context, int32_t id) { return context + " token id " + std::to_string(id); }

}  // namespace

CompactVocab::CompactVocab(const EngineConfig& config) {
    const Json cv = config.compact_vocab();
    enabled_ = cv.get_bool("enabled", false);
    if (!enabled_) return;

    reject_unknown_input_ids_ = cv.get_bool("reject_unknown_input_ids", true);
    check<ConfigurationError>(reject_unknown_input_ids_,
                              "compact_vocab v1 requires reject_unknown_input_ids=true because no unknown-token "
                              "remap is defined");
    mapping_path_ = resolve_mapping_path(config, cv.get_string("mapping_path"));
    const Json mapping = load_mapping(mapping_path_);
    check<ConfigurationError>(mapping.is_object() && mapping.get_string("format") == kCompactVocabFormat,
                              std::string("compact_vocab mapping format must be ") + kCompactVocabFormat);

    original_vocab_size_ = required_int(mapping, "original_vocab_size");
    compact_vocab_size_ = required_int(mapping, "compact_vocab_size");
    check<ConfigurationError>(original_vocab_size_ > 0, "original_vocab_size must be positive");
    check<ConfigurationError>(compact_vocab_size_ > 0, "compact_vocab_size must be positive");
    check<ConfigurationError>(compact_vocab_size_ <= original_vocab_size_,
                              "compact_vocab_size must be <= original_vocab_size");

    old_to_new_ = required_int_array(mapping, "old_to_new");
    new_to_old_ = required_int_array(mapping, "new_to_old");
    check<ConfigurationError>((int32_t)old_to_new_.size() == original_vocab_size_,
                              "old_to_new length must equal original_vocab_size");
    check<ConfigurationError>((int32_t)new_to_old_.size() == compact_vocab_size_,
                              "new_to_old length must equal compact_vocab_size");
    // the two tables must be inverse bijections on the kept ids (:124-143)
    for (int32_t o = 0; o < original_vocab_size_; ++o) {
        const int32_t n = old_to_new_[o];
        check<ConfigurationError>(n >= -1 && n < compact_vocab_size_,
                                  "old_to_new contains out-of-range compact id at original id " + std::to_string(o));
        if (n >= 0)
            check<ConfigurationError>(new_to_old_[n] == o,
                                      "old_to_new/new_to_old mismatch at original id " + std::to_string(o));
    }
    for (int32_t n = 0; n < compact_vocab_size_; ++n) {
        const int32_t o = new_to_old_[n];
        check<ConfigurationError>(o >= 0 && o < original_vocab_size_,
                                  "new_to_old contains out-of-range original id at compact id " + std::to_string(n));
        check<ConfigurationError>(old_to_new_[o] == n,
                                  "new_to_old/old_to_new mismatch at compact id " + std::to_string(n));
    }

    validate_model_vocab_size(config, compact_vocab_size_);
    (void)remap_required_token_ids(required_int_array(mapping, "special_token_ids"), "compact_vocab.special_token_ids");
    (void)remap_required_token_ids(config.eos_token_ids(), "model eos_token_ids");
    (void)remap_required_token_ids(config.stop_token_ids(), "sampling.stop_token_ids");
}

int32_t CompactVocab::remap_input_token_id(int32_t id, const std::string& context) const {
    if (!enabled_) return id;
    if (id < 0 || id >= original_vocab_size_ || old_to_new_[id] < 0)
        throw InvalidRequestError("compact_vocab cannot remap " + ids_context(context, id) +
                                  "; the token is absent from old_to_new");
    return old_to_new_[id];
}

int32_t CompactVocab::remap_required_token_id(int32_t id, const std::string& context) const {
    if (!enabled_) return id;
    check<ConfigurationError>(id >= 0 && id < original_vocab_size_ && old_to_new_[id] >= 0,
                              "compact_vocab requires " + ids_context(context, id) + " to be present in old_to_new");
    return old_to_new_[id];
}

int32_t CompactVocab::restore_token_id(int32_t id, const std::string& context) const {
    if (!enabled_) return id;
    if (id < 0 || id >= compact_vocab_size_)
        throw InternalError("compact_vocab cannot restore " + ids_context(context, id) + "; compact id is out of range");
    return new_to_old_[id];
}

std::vector<int32_t> CompactVocab::remap_token_ids(const std::vector<int32_t>& ids, const std::string& context) const {
    if (!enabled_) return ids;
    std::vector<int32_t> out;
    out.reserve(ids.size());
    for (int32_t id : ids) out.push_back(remap_input_token_id(id, context));
    return out;
}

std::vector<int32_t> CompactVocab::remap_required_token_ids(const std::vector<int32_t>& ids,
                                                            const std::string& context) const {
    if (!enabled_) return ids;
    std::vector<int32_t> out;
    out.reserve(ids.size());
    for (int32_t id : ids) out.push_back(remap_required_token_id(id, context));
    return out;
}

std::vector<int32_t> CompactVocab::remap_optional_token_ids(const std::vector<int32_t>& ids,
                                                            const std::string& context) const {
    return remap_required_token_ids(ids, context);
}

std::vector<int32_t> CompactVocab::restore_token_ids(const std::vector<int32_t>& ids, const std::string& context) const {
    if (!enabled_) return ids;
    std::vector<int32_t> out;
    out.reserve(ids.size());
    for (int32_t id : ids) out.push_back(restore_token_id(id, context));
    return out;
}

// Custom-embedding placeholders [base, base + rows) must stay one contiguous range in
// compact ids, because the embedding kernel selects rows by id - base (:245-272).
int32_t CompactVocab::remap_embed_token_id(const Request& request) const {
    if (!request.has_embedding() || request.embed_token_id < 0) return request.embed_token_id;
    const auto& shape = request.embedding.shape();
    check<InvalidRequestError>(!shape.empty() && shape[0] >= 0,
                               "compact_vocab requires embeddings to expose num_custom_embeddings in shape[0]");
    const int32_t rows = (int32_t)shape[0];
    const int32_t old_base = request.embed_token_id;
    const int32_t new_base = remap_input_token_id(old_base, "request embed_token_id");
    for (int32_t i = 0; i < rows; ++i) {
        const int32_t n = remap_input_token_id(old_base + i, "request embedding placeholder");
        if (n != new_base + i)
            throw InvalidRequestError(
                "compact_vocab requires custom embedding placeholder ids to remap to a contiguous range. old_base=" +
                std::to_string(old_base) + ", compact_base=" + std::to_string(new_base) + ", offset=" +
                std::to_string(i) + ", compact_id=" + std::to_string(n));
    }
    return new_base;
}

Request CompactVocab::remap_request(const Request& request) const {
    check<InvalidRequestError>(enabled_, "remap_request requires compact_vocab to be enabled");
    Request out(request.request_id, remap_token_ids(request.token_ids, "request token_ids"));
    out.embed_token_id = remap_embed_token_id(request);
    if (request.has_position_ids())
        check<InvalidRequestError>(request.has_embedding(),
                                   "compact_vocab VLM/custom position_ids requests require embeddings");
    out.embedding = request.embedding;
    out.position_ids = request.position_ids;
    out.mrope_last_pos = request.mrope_last_pos;
    out.stop_token_ids = remap_token_ids(request.stop_token_ids, "request stop_token_ids");
    out.ignore_stop_tokens = request.ignore_stop_tokens;
    return out;
}

}  // namespace edge_fm
