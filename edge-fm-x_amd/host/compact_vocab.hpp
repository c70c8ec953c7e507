// Compact vocabulary: the engine runs a pre-pruned checkpoint whose vocabulary holds
// only a subset of the original token ids (smaller embedding table and LM head, so
// the largest decode GEMV shrinks with it). Requests and responses stay in the
// original id space: input ids, custom-embedding placeholder ids, stop ids and the
// fixed KV prefixes are remapped old -> new on the way in, generated ids new -> old
// on the way out.
//
// Mirrors src/engine/tasks/token_generation/compact_vocab.{h,cpp} (class CompactVocab,
// mapping format "edgefm.compact_vocab.v1") with the same checks and error types.
#pragma once

#include <cstdint>
#include <string>
#include <vector>

#include "core.hpp"

namespace edge_fm {

class EngineConfig;

class CompactVocab {
public:
    CompactVocab() = default;
    // Reads config.compact_vocab() {enabled, mapping_path, reject_unknown_input_ids};
    // disabled (the default) makes every call an identity (compact_vocab.cpp:86-149).
    explicit CompactVocab(const EngineConfig& config);

    bool enabled() const noexcept { return enabled_; }
    int32_t original_vocab_size() const noexcept { return original_vocab_size_; }
    int32_t compact_vocab_size() const noexcept { return compact_vocab_size_; }
    const std::string& mapping_path() const noexcept { return mapping_path_; }

    // Request-side ids: an id outside old_to_new raises InvalidRequestError.
    std::vector<int32_t> remap_token_ids(const std::vector<int32_t>& ids, const std::string& context) const;
    // Configuration ids (EOS, stop ids, KV prefixes): a pruned id raises ConfigurationError.
    std::vector<int32_t> remap_required_token_ids(const std::vector<int32_t>& ids, const std::string& context) const;
    std::vector<int32_t> remap_optional_token_ids(const std::vector<int32_t>& ids, const std::string& context) const;
    // Generated ids back to the original space: out-of-range raises InternalError.
    std::vector<int32_t> restore_token_ids(const std::vector<int32_t>& ids, const std::string& context) const;
    // Copy of the request in compact ids (token ids, embed_token_id base, stop ids).
    Request remap_request(const Request& request) const;

private:
    int32_t remap_input_token_id(int32_t id, const std::string& context) const;
    int32_t remap_required_token_id(int32_t id, const std::string& context) const;
    int32_t restore_token_id(int32_t id, const std::string& context) const;
    int32_t remap_embed_token_id(const Request& request) const;

    bool enabled_ = false;
    bool reject_unknown_input_ids_ = true;
    int32_t original_vocab_size_ = 0;
    int32_t compact_vocab_size_ = 0;
    std::string mapping_path_;
    std::vector<int32_t> old_to_new_;
    std::vector<int32_t> new_to_old_;
};

}  // namespace edge_fm
