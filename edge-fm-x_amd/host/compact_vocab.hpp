// Compact vocabulary: a pre-pruned checkpoint keeps only a subset of the original token
// ids, so its embedding table and LM head are smaller (the LM head is the largest decode
// GEMV). Callers keep speaking original ids: everything that enters the engine (request
// ids, custom-embedding placeholder ids, stop / EOS ids, fixed KV prefixes) is translated
// original -> compact, and generated ids compact -> original on the way out.
//
// The public surface and the mapping file (format "edgefm.compact_vocab.v1": original and
// compact sizes, old_to_new with -1 for pruned ids, new_to_old, special_token_ids) are the
// reference's (src/engine/tasks/token_generation/compact_vocab.h); the implementation is a
// single validated id bijection plus one translation routine whose failure policy decides
// which error a caller sees.
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
    // Reads the engine config's compact_vocab section {enabled, mapping_path,
    // reject_unknown_input_ids}; disabled (the default) makes every translation the identity.
    explicit CompactVocab(const EngineConfig& config);

    bool enabled() const noexcept { return map_.active(); }
    int32_t original_vocab_size() const noexcept { return map_.original_size(); }
    int32_t compact_vocab_size() const noexcept { return map_.compact_size(); }
    const std::string& mapping_path() const noexcept { return path_; }

    // Request ids (original -> compact); an id with no compact slot is InvalidRequestError.
    std::vector<int32_t> remap_token_ids(const std::vector<int32_t>& ids, const std::string& context) const;
    // Configuration ids (EOS, stop ids, KV prefixes); a pruned id is ConfigurationError.
    std::vector<int32_t> remap_required_token_ids(const std::vector<int32_t>& ids, const std::string& context) const;
    std::vector<int32_t> remap_optional_token_ids(const std::vector<int32_t>& ids, const std::string& context) const;
    // Generated ids (compact -> original); an id outside the compact range is InternalError.
    std::vector<int32_t> restore_token_ids(const std::vector<int32_t>& ids, const std::string& context) const;
    // The request in compact ids (token ids, custom-embedding base id, stop ids).
    Request remap_request(const Request& request) const;

    // Which exception a failed translation raises.
    enum class OnMissing { Reject, Misconfigured, Corrupt };
    enum class Direction { ToCompact, ToOriginal };

private:
    // Two arrays that are inverse to each other on the kept ids: fwd (original -> compact,
    // -1 where pruned) and inv (compact -> original). An empty map is the identity.
    class IdBijection {
    public:
        void assign(std::vector<int32_t> fwd, std::vector<int32_t> inv);   // validates
        bool active() const noexcept { return !inv_.empty(); }
        int32_t original_size() const noexcept { return (int32_t)fwd_.size(); }
        int32_t compact_size() const noexcept { return (int32_t)inv_.size(); }
        // -1 when id has no image in that direction
        int32_t image(Direction d, int32_t id) const noexcept;

    private:
        std::vector<int32_t> fwd_, inv_;
    };

    int32_t translate(int32_t id, Direction d, OnMissing policy, const std::string& what) const;
    std::vector<int32_t> translate_all(const std::vector<int32_t>& ids, Direction d, OnMissing policy,
                                       const std::string& what) const;
    int32_t compact_embedding_base(const Request& request) const;

    IdBijection map_;
    std::string path_;
};

}  // namespace edge_fm
