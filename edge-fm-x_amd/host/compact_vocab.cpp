// Compact-vocabulary id translation (behaviour of the reference's
// src/engine/tasks/token_generation/compact_vocab.cpp; own implementation).
#include "compact_vocab.hpp"

#include <filesystem>
#include <utility>

#include "engine.hpp"
#include "json.hpp"

namespace fs = std::filesystem;

namespace edge_fm {

namespace {

const char* const kFormatTag = "edgefm.compact_vocab.v1";

// The integer fields of a v1 mapping file, read in one pass.
struct MappingFile {
    int64_t original_size = 0, compact_size = 0;
    std::vector<int32_t> old_to_new, new_to_old, special;
};

[[noreturn]] void bad_mapping(const std::string& path, const std::string& why) {
    throw ConfigurationError("compact vocabulary mapping " + path + ": " + why);
}

std::vector<int32_t> int_list(const Json& doc, const std::string& key, const std::string& path) {
    if (!doc.contains(key) || !doc.at(key).is_array()) bad_mapping(path, "'" + key + "' must be an array of integers");
    std::vector<int32_t> v;
    for (const Json& e : doc.at(key).as_array()) {
        if (!e.is_integer()) bad_mapping(path, "'" + key + "' holds a non-integer entry");
        v.push_back((int32_t)e.as_int());
    }
    return v;
}

int64_t int_field(const Json& doc, const std::string& key, const std::string& path) {
    if (!doc.contains(key) || !doc.at(key).is_integer()) bad_mapping(path, "'" + key + "' must be an integer");
    return doc.at(key).as_int();
}

MappingFile read_mapping(const std::string& path) {
    if (!fs::is_regular_file(path)) bad_mapping(path, "file not found");
    Json doc;
    try {
        doc = Json::parse_file(path);
    } catch (const std::exception& e) {
        bad_mapping(path, std::string("not valid JSON (") + e.what() + ")");
    }
    if (!doc.is_object() || doc.get_string("format") != kFormatTag)
        bad_mapping(path, std::string("'format' must be ") + kFormatTag);
    MappingFile m;
    m.original_size = int_field(doc, "original_vocab_size", path);
    m.compact_size = int_field(doc, "compact_vocab_size", path);
    if (m.original_size <= 0 || m.compact_size <= 0 || m.compact_size > m.original_size)
        bad_mapping(path, "sizes must satisfy 0 < compact_vocab_size <= original_vocab_size");
    m.old_to_new = int_list(doc, "old_to_new", path);
    m.new_to_old = int_list(doc, "new_to_old", path);
    m.special = int_list(doc, "special_token_ids", path);
    if ((int64_t)m.old_to_new.size() != m.original_size || (int64_t)m.new_to_old.size() != m.compact_size)
        bad_mapping(path, "old_to_new / new_to_old lengths must equal the two vocabulary sizes");
    return m;
}

// vocab_size of the checkpoint the engine loads (Qwen2.5-VL keeps it under text_config).
int64_t checkpoint_vocab(const EngineConfig& config) {
    const Json& mc = config.model_config();
    const Json& src = (!mc.contains("vocab_size") && mc.contains("text_config")) ? mc.at("text_config") : mc;
    if (!src.contains("vocab_size") || !src.at("vocab_size").is_integer())
        throw ConfigurationError("compact vocabulary: the model config has no integer vocab_size");
    return src.at("vocab_size").as_int();
}

}  // namespace

void CompactVocab::IdBijection::assign(std::vector<int32_t> fwd, std::vector<int32_t> inv) {
    // each array must land inside the other's index range and come back to where it started
    auto round_trips = [](const std::vector<int32_t>& there, const std::vector<int32_t>& back, bool holes,
                          const char* name) {
        for (size_t i = 0; i < there.size(); ++i) {
            const int32_t t = there[i];
            if (holes && t == -1) continue;
            if (t < 0 || (size_t)t >= back.size() || back[(size_t)t] != (int32_t)i)
                throw ConfigurationError(std::string("compact vocabulary: ") + name + "[" + std::to_string(i) +
                                         "] = " + std::to_string(t) + " is not inverted by the other table");
        }
    };
    round_trips(fwd, inv, true, "old_to_new");
    round_trips(inv, fwd, false, "new_to_old");
    fwd_ = std::move(fwd);
    inv_ = std::move(inv);
}

int32_t CompactVocab::IdBijection::image(Direction d, int32_t id) const noexcept {
    const std::vector<int32_t>& table = (d == Direction::ToCompact) ? fwd_ : inv_;
    return (id >= 0 && (size_t)id < table.size()) ? table[(size_t)id] : -1;
}

CompactVocab::CompactVocab(const EngineConfig& config) {
    const Json section = config.compact_vocab();
    if (!section.get_bool("enabled", false)) return;
    // v1 defines no replacement for ids missing from the mapping, so they must be rejected
    if (!section.get_bool("reject_unknown_input_ids", true))
        throw ConfigurationError("compact vocabulary v1 supports only reject_unknown_input_ids = true");
    const std::string raw = section.get_string("mapping_path");
    if (raw.empty()) throw ConfigurationError("compact vocabulary is enabled but compact_vocab.mapping_path is empty");
    fs::path p(raw);
    if (p.is_relative()) p = fs::path(config.config_dir()) / p;   // relative to the engine config
    path_ = p.lexically_normal().string();

    MappingFile m = read_mapping(path_);
    if (checkpoint_vocab(config) != m.compact_size)
        throw ConfigurationError("compact vocabulary v1 needs the pruned checkpoint: model vocab_size " +
                                 std::to_string(checkpoint_vocab(config)) + " differs from compact_vocab_size " +
                                 std::to_string(m.compact_size));
    map_.assign(std::move(m.old_to_new), std::move(m.new_to_old));
    // every id the engine itself depends on must survive the pruning
    translate_all(m.special, Direction::ToCompact, OnMissing::Misconfigured, "special token");
    translate_all(config.eos_token_ids(), Direction::ToCompact, OnMissing::Misconfigured, "EOS token");
    translate_all(config.stop_token_ids(), Direction::ToCompact, OnMissing::Misconfigured, "configured stop token");
}

int32_t CompactVocab::translate(int32_t id, Direction d, OnMissing policy, const std::string& what) const {
    if (!map_.active()) return id;
    const int32_t out = map_.image(d, id);
    if (out >= 0) return out;
    const std::string msg = "compact vocabulary: " + what + " " + std::to_string(id) +
                            (d == Direction::ToCompact ? " was pruned from (or lies outside) the original vocabulary"
                                                       : " is not a compact id");
    switch (policy) {
        case OnMissing::Reject: throw InvalidRequestError(msg);
        case OnMissing::Misconfigured: throw ConfigurationError(msg);
        case OnMissing::Corrupt: throw InternalError(msg);
    }
    throw InternalError(msg);
}

std::vector<int32_t> CompactVocab::translate_all(const std::vector<int32_t>& ids, Direction d, OnMissing policy,
                                                 const std::string& what) const {
    std::vector<int32_t> out(ids.size());
    for (size_t i = 0; i < ids.size(); ++i) out[i] = translate(ids[i], d, policy, what);
    return out;
}

std::vector<int32_t> CompactVocab::remap_token_ids(const std::vector<int32_t>& ids, const std::string& context) const {
    return translate_all(ids, Direction::ToCompact, OnMissing::Reject, context);
}

std::vector<int32_t> CompactVocab::remap_required_token_ids(const std::vector<int32_t>& ids,
                                                            const std::string& context) const {
    return translate_all(ids, Direction::ToCompact, OnMissing::Misconfigured, context);
}

std::vector<int32_t> CompactVocab::remap_optional_token_ids(const std::vector<int32_t>& ids,
                                                            const std::string& context) const {
    return translate_all(ids, Direction::ToCompact, OnMissing::Misconfigured, context);
}

std::vector<int32_t> CompactVocab::restore_token_ids(const std::vector<int32_t>& ids, const std::string& context) const {
    return translate_all(ids, Direction::ToOriginal, OnMissing::Corrupt, context);
}

// The embedding kernel picks custom rows by (id - base), so the placeholder ids
// [base, base + rows) must still be consecutive after translation.
int32_t CompactVocab::compact_embedding_base(const Request& request) const {
    if (!request.has_embedding() || request.embed_token_id < 0) return request.embed_token_id;
    const auto& shape = request.embedding.shape();
    if (shape.empty() || shape[0] < 0)
        throw InvalidRequestError("compact vocabulary: custom embeddings need their row count in shape[0]");
    const int32_t base = translate(request.embed_token_id, Direction::ToCompact, OnMissing::Reject,
                                   "custom-embedding base id");
    for (int64_t row = 1; row < shape[0]; ++row) {
        const int32_t id = request.embed_token_id + (int32_t)row;
        if (translate(id, Direction::ToCompact, OnMissing::Reject, "custom-embedding placeholder id") !=
            base + (int32_t)row)
            throw InvalidRequestError("compact vocabulary: custom-embedding placeholder " + std::to_string(id) +
                                      " does not stay consecutive with base " +
                                      std::to_string(request.embed_token_id) + " after translation");
    }
    return base;
}

Request CompactVocab::remap_request(const Request& request) const {
    if (!map_.active()) throw InvalidRequestError("remap_request called with the compact vocabulary disabled");
    if (request.has_position_ids() && !request.has_embedding())
        throw InvalidRequestError("compact vocabulary: position_ids are accepted only with custom embeddings");
    Request out(request.request_id, remap_token_ids(request.token_ids, "request token id"));
    out.embed_token_id = compact_embedding_base(request);
    out.embedding = request.embedding;
    out.position_ids = request.position_ids;
    out.mrope_last_pos = request.mrope_last_pos;
    out.stop_token_ids = remap_token_ids(request.stop_token_ids, "request stop token id");
    out.ignore_stop_tokens = request.ignore_stop_tokens;
    return out;
}

}  // namespace edge_fm
