"""Prefill HIP graphs (standard_engine.cpp:568-800 of the reference: one graph per
(request, prefill length), captured once and replayed with the request's ids refreshed).
Here the first prefill of a key runs eagerly, the second is captured and replayed, later
ones replay; a replay must reproduce the eager engine exactly: the same tokens and the
same fp32 logits bit for bit (the same kernels on the same inputs), for new ids of the
same length, after a longer prompt has grown the prefill buffers (the graph is then
captured again), for a fixed-prefix slot (cache base > 0) and for Qwen2.5-VL requests
whose custom embedding rows and M-RoPE positions change between calls."""
import os
import tempfile

import numpy as np
import pytest
import torch

import edge_fm
import efm_setup as S
from oracle import efm_oracle as O

pytestmark = pytest.mark.gpu

TINY = S.ModelShape(hidden=256, layers=2, heads=4, kv_heads=2, head_dim=64, inter=512, vocab=1000)
TINY_VL = S.ModelShape(hidden=256, layers=2, heads=4, kv_heads=2, head_dim=64, inter=512, vocab=1000,
                       mrope_section=(8, 12, 12))


def _cfg(shape):
    return O.QwenConfig(hidden=shape.hidden, layers=shape.layers, heads=shape.heads, kv_heads=shape.kv_heads,
                        head_dim=shape.head_dim, inter=shape.inter, vocab=shape.vocab, tied=shape.tied,
                        mrope_section=shape.mrope_section)


def _engines(tmp, shape, w, **cfg):
    """A graph engine and an eager engine over the same weights (both fuse their own copy
    at construction, so the registered tensors may be replaced in between)."""
    out = []
    for g in (True, False):
        wdev = {k: v.to("cuda:0").contiguous() for k, v in w.items()}
        S.register_weights(wdev)
        mdir = S.write_model_dir(os.path.join(tmp, f"model_{g}"), shape)
        ecfg = S.write_engine_config(os.path.join(tmp, f"engine_{g}.json"), mdir, use_graph=g, debug_logits=True,
                                     **cfg)
        out.append((edge_fm.EdgeFM(ecfg), wdev))
    return out


def _run(eng, req):
    toks = eng.generate(req).token_ids()
    return toks, np.array(eng.last_logits()), eng.last_generate_metrics()


def _req(ids):
    r = edge_fm.Request(0, list(ids))
    r.set_ignore_stop_tokens(True)
    return r


def test_prefill_graph_replays_equal_eager_prefill():
    w = O.random_weights(_cfg(TINY), seed=21, std=0.2)
    g = torch.Generator().manual_seed(4)
    A = torch.randint(0, TINY.vocab, (40,), generator=g).tolist()
    B = torch.randint(0, TINY.vocab, (40,), generator=g).tolist()
    C = torch.randint(0, TINY.vocab, (100,), generator=g).tolist()   # grows the prefill buffers
    with tempfile.TemporaryDirectory() as tmp:
        (ge, _k1), (ee, _k2) = _engines(tmp, TINY, w, max_tokens=160, max_new_tokens=16)
        ref = {name: _run(ee, _req(p)) for name, p in (("A", A), ("B", B), ("C", C))}
        # (prompt, replayed?) : first A eager, then captured; B reuses A's graph with new
        # ids; C eager (new key); A again is captured anew (C replaced the buffers)
        plan = [("A", False), ("A", True), ("B", True), ("C", False), ("A", True), ("B", True), ("C", True)]
        for i, (name, replayed) in enumerate(plan):
            toks, logits, m = _run(ge, _req({"A": A, "B": B, "C": C}[name]))
            assert m["prefill_graph_replayed"] == (1.0 if replayed else 0.0), f"call {i} ({name})"
            assert toks == ref[name][0], f"call {i} ({name}): tokens differ from the eager engine"
            assert np.array_equal(logits, ref[name][1]), f"call {i} ({name}): logits differ from the eager engine"
        assert ee.last_generate_metrics()["prefill_graph_replayed"] == 0.0


def test_prefill_graph_with_fixed_prefix_slot():
    w = O.random_weights(_cfg(TINY), seed=22, std=0.2)
    prefix = list(range(3, 19))
    tails = [[50, 51, 52, 53, 54, 55, 56, 57], [60, 61, 62, 63, 64, 65, 66, 67], [70, 71, 72, 73, 74, 75, 76, 77]]
    with tempfile.TemporaryDirectory() as tmp:
        (ge, _k1), (ee, _k2) = _engines(tmp, TINY, w, max_tokens=96, max_new_tokens=10, prefix_token_ids=prefix)
        for i, t in enumerate(tails):
            toks, logits, m = _run(ge, _req(prefix + t))
            etoks, elogits, _ = _run(ee, _req(prefix + t))
            assert m["prefill_tokens"] == len(t), "only the suffix after the prefix is prefilled"
            assert m["prefill_graph_replayed"] == (0.0 if i == 0 else 1.0)
            assert toks == etoks and np.array_equal(logits, elogits), f"suffix {i}"


def test_prefill_graph_vl_embeddings_and_positions_change():
    shape = TINY_VL
    w = O.random_weights(_cfg(shape), seed=23, std=0.2)
    n_vis, n_txt, eid = 24, 8, 900
    ids = [eid + i for i in range(n_vis)] + list(range(10, 10 + n_txt))

    def request(seed, shift):
        vis = torch.randn(n_vis, shape.hidden, generator=torch.Generator().manual_seed(seed)).to(torch.bfloat16)
        t = torch.zeros(n_vis, dtype=torch.int32) + shift
        hh = torch.arange(n_vis, dtype=torch.int32) // 6 + shift
        ww = torch.arange(n_vis, dtype=torch.int32) % 6 + shift
        start = int(max(hh.max(), ww.max())) + 1
        txt = torch.arange(start, start + n_txt, dtype=torch.int32)
        pos = torch.stack([torch.cat([t, txt]), torch.cat([hh, txt]), torch.cat([ww, txt])]).contiguous()
        vis_g, pos_g = vis.to("cuda:0"), pos.to("cuda:0")
        r = edge_fm.Request(0, ids, edge_fm.Tensor(vis_g.data_ptr(), list(vis_g.shape), edge_fm.DType.BFloat16,
                                                   edge_fm.Device.GPU, 0, False), eid,
                            edge_fm.Tensor(pos_g.data_ptr(), [3, len(ids)], edge_fm.DType.Int32, edge_fm.Device.GPU, 0,
                                           False))
        r.set_ignore_stop_tokens(True)
        return r, (vis_g, pos_g)

    with tempfile.TemporaryDirectory() as tmp:
        (ge, _k1), (ee, _k2) = _engines(tmp, shape, w, max_tokens=96, max_new_tokens=10, model_name="qwen2_5_vl")
        for i, (seed, shift) in enumerate([(1, 0), (2, 3), (3, 1), (1, 0)]):
            r, keep = request(seed, shift)
            toks, logits, m = _run(ge, r)
            etoks, elogits, _ = _run(ee, r)
            assert m["prefill_graph_replayed"] == (0.0 if i == 0 else 1.0)
            assert toks == etoks and np.array_equal(logits, elogits), f"call {i}"


@pytest.mark.parametrize("prompt_len,gen,max_tokens", [(100, 200, 400), (1000, 60, 1100)])
def test_decode_graphs_per_row_bucket_equal_eager(prompt_len, gen, max_tokens):
    """Decode graphs are captured per 128-row bucket of the lengths their steps reach
    (StandardEngine::decode_row_bound): generations that cross buckets inside an 8-step
    graph, and (1000 + 60 rows) cross from the 8-split plan whose merge folds into o_proj
    (<= 1024 rows) to the generic attention, must equal the eager engine's tokens and fp32
    logits bit for bit."""
    w = O.random_weights(_cfg(TINY), seed=24, std=0.2)
    ids = torch.randint(0, TINY.vocab, (prompt_len,), generator=torch.Generator().manual_seed(9)).tolist()
    with tempfile.TemporaryDirectory() as tmp:
        (ge, _k1), (ee, _k2) = _engines(tmp, TINY, w, max_tokens=max_tokens, max_new_tokens=gen)
        etoks, elogits, _ = _run(ee, _req(ids))
        for rep in range(2):
            toks, logits, m = _run(ge, _req(ids))
            assert len(toks) == gen and m["decode_steps"] == gen - 1
            assert toks == etoks, f"rep {rep}: tokens differ from the eager engine"
            assert np.array_equal(logits, elogits), f"rep {rep}: logits differ from the eager engine"
