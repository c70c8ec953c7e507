"""Compact-vocabulary id mapping (host only, no GPU): the cases of the reference's
tests/cpp/test_compact_vocab.cpp (non-identity remap/restore, disabled no-op, identity
request, request stop-id remap, unknown input rejected, pruned request stop id
rejected) plus the configuration checks of compact_vocab.cpp:86-149, all through the
pybind `edge_fm.CompactVocab` built from an engine config file."""
import json
import os

import pytest

import edge_fm
import efm_setup as S

SMALL = dict(hidden=8, layers=1, heads=1, kv_heads=1, head_dim=8, inter=16)


def _config(tmp_path, vocab, compact=None, mapping=None, stop_ids=None, eos=None, prefix=None):
    mdir = S.write_model_dir(str(tmp_path / "model"), S.ModelShape(**SMALL, vocab=vocab), eos_token_id=eos)
    if mapping is not None:
        with open(tmp_path / "compact_vocab.json", "w") as f:
            json.dump(mapping, f)
    return S.write_engine_config(str(tmp_path / "engine.json"), mdir, max_tokens=8, stop_token_ids=stop_ids,
                                 compact_vocab=compact, prefix_token_ids=prefix)


def _mapping(original, new_to_old, special, fmt="edgefm.compact_vocab.v1"):
    old_to_new = [-1] * original
    for n, o in enumerate(new_to_old):
        old_to_new[o] = n
    return {"format": fmt, "original_vocab_size": original, "compact_vocab_size": len(new_to_old),
            "old_to_new": old_to_new, "new_to_old": list(new_to_old), "special_token_ids": list(special)}


ENABLED = {"enabled": True, "mapping_path": "compact_vocab.json", "reject_unknown_input_ids": True}
PERM = _mapping(6, [3, 4, 1], [1, 3])  # old_to_new = [-1, 2, -1, 0, 1, -1]


def test_mapping_file_layout_matches_reference_case(tmp_path):
    assert PERM["old_to_new"] == [-1, 2, -1, 0, 1, -1]
    p = S.write_compact_vocab_mapping(str(tmp_path / "m.json"), 6, [3, 4, 1], [1, 3])
    with open(p) as f:
        assert json.load(f) == PERM


def test_non_identity_remap_and_restore(tmp_path):
    cv = edge_fm.CompactVocab(_config(tmp_path, 3, ENABLED, PERM))
    assert cv.enabled() and cv.compact_vocab_size() == 3 and cv.original_vocab_size() == 6
    internal = cv.remap_token_ids([3, 4, 1], "request token_ids")
    assert internal == [0, 1, 2]
    assert cv.restore_token_ids(internal, "response token_ids") == [3, 4, 1]
    assert cv.remap_required_token_ids([1, 3], "stop_token_ids") == [2, 0]
    assert os.path.samefile(cv.mapping_path(), tmp_path / "compact_vocab.json")


def test_disabled_mapping_is_noop(tmp_path):
    cv = edge_fm.CompactVocab(_config(tmp_path, 8))
    assert not cv.enabled()
    ids = [0, 7, 3, 12345, -4]
    assert cv.remap_token_ids(ids, "request token_ids") == ids
    assert cv.restore_token_ids(ids, "response token_ids") == ids
    assert cv.remap_required_token_ids(ids, "x") == ids
    with pytest.raises(edge_fm.InvalidRequestError):
        cv.remap_request(edge_fm.Request(0, [1]))


def test_identity_mapping_request_remap(tmp_path):
    cv = edge_fm.CompactVocab(_config(tmp_path, 4, ENABLED, _mapping(4, [0, 1, 2, 3], [0, 3]), stop_ids=[3]))
    req = edge_fm.Request(0, [0, 1, 2])
    req.set_stop_token_ids([3])
    r = cv.remap_request(req)
    assert r.token_ids() == [0, 1, 2] and r.stop_token_ids() == [3]
    assert cv.restore_token_ids(r.token_ids(), "response token_ids") == [0, 1, 2]


def test_non_identity_request_stop_remap(tmp_path):
    cv = edge_fm.CompactVocab(_config(tmp_path, 3, ENABLED, PERM))
    req = edge_fm.Request(5, [3, 4, 1])
    req.set_stop_token_ids([1])
    req.set_ignore_stop_tokens(True)
    r = cv.remap_request(req)
    assert r.request_id() == 5 and r.token_ids() == [0, 1, 2] and r.stop_token_ids() == [2]
    assert r.ignore_stop_tokens()
    assert cv.restore_token_ids(r.token_ids(), "response token_ids") == [3, 4, 1]


def test_unknown_input_rejected(tmp_path):
    cv = edge_fm.CompactVocab(_config(tmp_path, 2, ENABLED, _mapping(4, [0, 2], [0])))
    for bad in ([0, 1, 2], [4], [-1]):
        with pytest.raises(edge_fm.InvalidRequestError):
            cv.remap_token_ids(bad, "request token_ids")
    with pytest.raises(edge_fm.InternalError):
        cv.restore_token_ids([2], "response token_ids")


def test_remap_request_rejects_pruned_stop_token(tmp_path):
    cv = edge_fm.CompactVocab(_config(tmp_path, 2, ENABLED, _mapping(4, [0, 2], [0])))
    req = edge_fm.Request(0, [0, 2])
    req.set_stop_token_ids([3])
    with pytest.raises(edge_fm.InvalidRequestError):
        cv.remap_request(req)


def test_custom_embedding_placeholders_must_stay_contiguous(tmp_path):
    import torch

    emb = torch.zeros(2, 8, dtype=torch.bfloat16)
    t = edge_fm.Tensor(emb.data_ptr(), [2, 8], edge_fm.DType.BFloat16, edge_fm.Device.CPU, 0)
    # original ids 4, 5 -> compact 1, 2 (contiguous)
    cv = edge_fm.CompactVocab(_config(tmp_path, 3, ENABLED, _mapping(6, [0, 4, 5], [0])))
    r = cv.remap_request(edge_fm.Request(0, [0, 4, 5], t, 4))
    assert r.embed_token_id() == 1 and r.token_ids() == [0, 1, 2]
    # original ids 4, 5 -> compact 2, 1 (reversed): rejected
    cv = edge_fm.CompactVocab(_config(tmp_path, 3, ENABLED, _mapping(6, [0, 5, 4], [0])))
    with pytest.raises(edge_fm.InvalidRequestError):
        cv.remap_request(edge_fm.Request(0, [0, 4, 5], t, 4))
    # M-RoPE position ids without embeddings: rejected
    pos = torch.zeros(3, 3, dtype=torch.int32)
    tp = edge_fm.Tensor(pos.data_ptr(), [3, 3], edge_fm.DType.Int32, edge_fm.Device.CPU, 0)
    empty = edge_fm.Tensor()
    with pytest.raises(edge_fm.InvalidRequestError):
        cv.remap_request(edge_fm.Request(0, [0, 4, 5], empty, -1, tp))


@pytest.mark.parametrize("case", [
    "no_path", "missing_file", "bad_json", "bad_format", "allow_unknown", "size_order", "len_mismatch",
    "inconsistent", "out_of_range", "model_vocab", "special_pruned", "eos_pruned", "stop_pruned", "float_entry",
])
def test_configuration_errors(tmp_path, case):
    mapping, compact, kw = dict(PERM), dict(ENABLED), {}
    vocab = 3
    if case == "no_path":
        compact["mapping_path"] = ""
    elif case == "missing_file":
        compact["mapping_path"] = "absent.json"
    elif case == "bad_format":
        mapping["format"] = "edgefm.compact_vocab.v0"
    elif case == "allow_unknown":
        compact["reject_unknown_input_ids"] = False
    elif case == "size_order":
        mapping["compact_vocab_size"] = 7
    elif case == "len_mismatch":
        mapping["new_to_old"] = [3, 4]
    elif case == "inconsistent":
        mapping["new_to_old"] = [4, 3, 1]
    elif case == "out_of_range":
        mapping["old_to_new"] = [-2, 2, -1, 0, 1, -1]
    elif case == "model_vocab":
        vocab = 6
    elif case == "special_pruned":
        mapping["special_token_ids"] = [2]
    elif case == "eos_pruned":
        kw["eos"] = 5
    elif case == "stop_pruned":
        kw["stop_ids"] = [0]
    elif case == "float_entry":
        mapping["new_to_old"] = [3.0, 4, 1]
    path = _config(tmp_path, vocab, compact, mapping, **kw)
    if case == "bad_json":
        with open(tmp_path / "compact_vocab.json", "w") as f:
            f.write("{not json")
    with pytest.raises(edge_fm.ConfigurationError):
        edge_fm.CompactVocab(path)


def test_eos_and_stop_ids_in_mapping_are_accepted(tmp_path):
    cv = edge_fm.CompactVocab(_config(tmp_path, 3, ENABLED, PERM, stop_ids=[4], eos=1))
    assert cv.remap_required_token_ids([4, 1], "x") == [1, 2]
