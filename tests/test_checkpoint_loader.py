"""The safetensors checkpoint path (src/utils/device/weight_loader.cpp:80-150,
src/engine/engine_factory.cpp:27-109): file collection, header parsing, the Qwen2.5-VL
key mapping (CPU), and loading a model through EdgeFM(config) from one file, from two
shards and from a VL-prefixed checkpoint with a vision tower, checked against the run
with the same tensors registered directly (GPU)."""
import json
import os
import struct
import tempfile

import pytest
import torch

import edge_fm
import efm_setup as S
from oracle import efm_oracle as O

TINY = S.ModelShape(hidden=256, layers=2, heads=4, kv_heads=2, head_dim=64, inter=512, vocab=1000)
TINY_UNTIED = S.ModelShape(hidden=256, layers=2, heads=4, kv_heads=2, head_dim=64, inter=512, vocab=1000, tied=False)
TINY_VL = S.ModelShape(hidden=256, layers=2, heads=4, kv_heads=2, head_dim=64, inter=512, vocab=1000,
                       mrope_section=(8, 12, 12))


def _weights(shape, seed):
    cfg = O.QwenConfig(hidden=shape.hidden, layers=shape.layers, heads=shape.heads, kv_heads=shape.kv_heads,
                       head_dim=shape.head_dim, inter=shape.inter, vocab=shape.vocab, tied=shape.tied,
                       mrope_section=shape.mrope_section)
    w = O.random_weights(cfg, seed=seed, std=0.2)
    if not shape.tied and "lm_head.weight" not in w:
        w["lm_head.weight"] = (torch.randn(shape.vocab, shape.hidden, generator=torch.Generator().manual_seed(seed))
                               * 0.2).to(torch.bfloat16)
    return w


# ------------------------------------------------------------------ CPU: host-side pieces
def test_header_matches_what_safetensors_wrote():
    w = _weights(TINY, 1)
    with tempfile.TemporaryDirectory() as tmp:
        (path,) = S.write_checkpoint(tmp, w)
        entries, data_off = edge_fm.read_safetensors_header(path)
        with open(path, "rb") as f:
            n = struct.unpack("<Q", f.read(8))[0]
            raw = json.loads(f.read(n))
        assert data_off == 8 + n
        assert set(entries) == set(w)
        for name, t in w.items():
            dtype, shape, begin, end = entries[name]
            assert dtype == "BF16" and list(shape) == list(t.shape)
            assert [begin, end] == raw[name]["data_offsets"]
            assert end - begin == t.numel() * 2


def test_collect_files_single_shards_and_errors():
    w = _weights(TINY, 2)
    with tempfile.TemporaryDirectory() as tmp:
        one = os.path.join(tmp, "one")
        (single,) = S.write_checkpoint(one, w)
        assert edge_fm.collect_safetensors_files(one) == [single]
        assert edge_fm.collect_safetensors_files(single) == [single]
        two = os.path.join(tmp, "two")
        shards = S.write_checkpoint(two, w, shards=2)
        # files that are not model-*-of-*.safetensors shards are ignored
        for junk in ("model-extra.safetensors", "optimizer.safetensors", "model-00001-of-00002.bin"):
            open(os.path.join(two, junk), "wb").close()
        assert edge_fm.collect_safetensors_files(two) == sorted(shards)
        assert [os.path.basename(p) for p in shards] == ["model-00001-of-00002.safetensors",
                                                          "model-00002-of-00002.safetensors"]
        # every tensor is in exactly one shard
        seen = []
        for p in shards:
            seen += list(edge_fm.read_safetensors_header(p)[0])
        assert sorted(seen) == sorted(w)
        empty = os.path.join(tmp, "empty")
        os.makedirs(empty)
        with pytest.raises(edge_fm.ConfigurationError):
            edge_fm.collect_safetensors_files(empty)


def test_malformed_headers_rejected():
    with tempfile.TemporaryDirectory() as tmp:
        def write(name, blob):
            p = os.path.join(tmp, name)
            with open(p, "wb") as f:
                f.write(blob)
            return p

        hdr = json.dumps({"a": {"dtype": "BF16", "shape": [2], "data_offsets": [0, 4]}}).encode()
        good = write("good.safetensors", struct.pack("<Q", len(hdr)) + hdr + b"\0" * 4)
        assert edge_fm.read_safetensors_header(good)[0]["a"][0] == "BF16"
        bad = {
            "short.safetensors": struct.pack("<Q", len(hdr) + 100) + hdr,          # header runs past the file
            "zero.safetensors": struct.pack("<Q", 0),
            "json.safetensors": struct.pack("<Q", 5) + b"{oops",
            "keys.safetensors": struct.pack("<Q", 14) + b'{"a": {"x": 1}',
        }
        neg = json.dumps({"a": {"dtype": "BF16", "shape": [2], "data_offsets": [4, 0]}}).encode()
        bad["order.safetensors"] = struct.pack("<Q", len(neg)) + neg
        for name, blob in bad.items():
            with pytest.raises(edge_fm.ModelNotLoadedError):
                edge_fm.read_safetensors_header(write(name, blob))


def test_vl_language_model_names():
    m = edge_fm.vl_language_model_name
    assert m("model.language_model.layers.3.mlp.up_proj.weight") == "model.layers.3.mlp.up_proj.weight"
    assert m("model.language_model.embed_tokens.weight") == "model.embed_tokens.weight"
    assert m("model.model.norm.weight") == "model.norm.weight"
    assert m("language_model.model.layers.0.input_layernorm.weight") == "model.layers.0.input_layernorm.weight"
    assert m("language_model.lm_head.weight") == "lm_head.weight"
    assert m("model.layers.0.self_attn.q_proj.bias") == "model.layers.0.self_attn.q_proj.bias"
    assert m("lm_head.weight") == "lm_head.weight"
    assert m("visual.blocks.0.attn.qkv.weight") == ""
    assert m("model.visual.patch_embed.proj.weight") == ""


# ------------------------------------------------------------------ GPU: through EdgeFM
def _generate(tmp, shape, model_dir, registered, model_name="", request=None):
    loader = edge_fm.WeightLoader.instance()
    loader.clear_stage(edge_fm.ModelStage.Prefill)
    if registered is not None:
        S.register_weights(registered)
    S.write_model_dir(model_dir, shape)
    ecfg = S.write_engine_config(os.path.join(tmp, "engine.json"), model_dir, max_tokens=96, max_new_tokens=16,
                                 model_name=model_name)
    eng = edge_fm.EdgeFM(ecfg)
    req = request() if request else edge_fm.Request(0, list(range(20, 52)))
    req.set_ignore_stop_tokens(True)
    toks = eng.generate(req).token_ids()
    names = set(loader.get(edge_fm.ModelStage.Prefill))
    del eng
    loader.clear_stage(edge_fm.ModelStage.Prefill)
    return toks, names


@pytest.mark.gpu
@pytest.mark.parametrize("shape", [TINY, TINY_UNTIED], ids=["tied", "untied"])
def test_engine_loads_single_file_and_shards(gpu, shape):
    w = _weights(shape, 3)
    wdev = {k: v.to(gpu).contiguous() for k, v in w.items()}
    with tempfile.TemporaryDirectory() as tmp:
        ref, _ = _generate(tmp, shape, os.path.join(tmp, "reg"), wdev)
        for shards in (1, 2):
            d = os.path.join(tmp, f"ckpt{shards}")
            S.write_checkpoint(d, w, shards=shards)
            toks, names = _generate(tmp, shape, d, None)
            assert names == set(w), f"{shards} shard(s): loaded tensor names differ"
            assert toks == ref, f"{shards} shard(s): tokens differ from the registered-tensor run"


@pytest.mark.gpu
def test_engine_loads_vl_prefixed_checkpoint(gpu):
    """Qwen2.5-VL layout: language model under model.language_model., head at lm_head.,
    plus vision-tower tensors that must not be loaded; custom embedding rows and M-RoPE
    positions as in a multimodal request."""
    shape = TINY_VL
    w = _weights(shape, 4)
    wdev = {k: v.to(gpu).contiguous() for k, v in w.items()}
    vis = torch.randn(12, shape.hidden, generator=torch.Generator().manual_seed(5)).to(torch.bfloat16).to(gpu)
    ids = [900 + i for i in range(12)] + list(range(30, 38))
    t = torch.zeros(12, dtype=torch.int32)
    hh, ww = torch.arange(12, dtype=torch.int32) // 4, torch.arange(12, dtype=torch.int32) % 4
    txt = torch.arange(4, 12, dtype=torch.int32)
    pos = torch.stack([torch.cat([t, txt]), torch.cat([hh, txt]), torch.cat([ww, txt])]).contiguous().to(gpu)

    def request():
        return edge_fm.Request(0, ids, edge_fm.Tensor(vis.data_ptr(), list(vis.shape), edge_fm.DType.BFloat16,
                                                      edge_fm.Device.GPU, 0, False), 900,
                               edge_fm.Tensor(pos.data_ptr(), [3, len(ids)], edge_fm.DType.Int32,
                                              edge_fm.Device.GPU, 0, False))

    def vl_name(k):
        return "model.language_model." + k[len("model."):] if k.startswith("model.") else k

    extra = {"model.visual.patch_embed.proj.weight": torch.randn(64, 48).to(torch.bfloat16),
             "visual.blocks.0.attn.qkv.weight": torch.randn(96, 32).to(torch.bfloat16)}
    with tempfile.TemporaryDirectory() as tmp:
        ref, _ = _generate(tmp, shape, os.path.join(tmp, "reg"), wdev, model_name="qwen2_5_vl", request=request)
        d = os.path.join(tmp, "vl")
        S.write_checkpoint(d, w, shards=2, rename=vl_name, extra=extra)
        toks, names = _generate(tmp, shape, d, None, model_name="qwen2_5_vl", request=request)
    assert names == set(w), "VL checkpoint: the language model's tensors under their text names, no vision tower"
    assert toks == ref
