"""End-to-end GPU tests of the C++ engine (pybind `edge_fm.EdgeFM.generate`) against
the CPU oracle: greedy token ids are compared step by step with the oracle
teacher-forced on the GPU's own tokens, so a mismatch is accepted only where the
oracle's top-1 / chosen-token logit gap is below the bf16 accumulation noise (a
near-tie flip). Mirrors tests/engine/test_qwen2_generate.py of the
reference (HF transformers dumps there; the oracle here is pinned to HF in
tests/test_oracle.py)."""
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


def _oracle_cfg(shape: S.ModelShape) -> O.QwenConfig:
    return O.QwenConfig(hidden=shape.hidden, layers=shape.layers, heads=shape.heads, kv_heads=shape.kv_heads,
                        head_dim=shape.head_dim, inter=shape.inter, vocab=shape.vocab, eps=shape.eps,
                        theta=shape.theta, tied=shape.tied, mrope_section=shape.mrope_section)


def _engine(tmp, shape, weights_cpu, **cfg):
    wdev = {k: v.to("cuda:0").contiguous() for k, v in weights_cpu.items()}
    S.register_weights(wdev)
    mdir = S.write_model_dir(os.path.join(tmp, "model"), shape)
    ecfg = S.write_engine_config(os.path.join(tmp, "engine.json"), mdir, **cfg)
    return edge_fm.EdgeFM(ecfg), wdev


def _check_against_oracle(tokens, steps, tol):
    assert len(tokens) == len(steps)
    exact = 0
    for i, (tok, (ref, margin, gap)) in enumerate(zip(tokens, steps)):
        if tok == ref:
            exact += 1
        else:
            assert gap < tol, f"step {i}: gpu {tok} vs oracle {ref}, logit gap {gap:.4f} (margin {margin:.4f})"
    return exact


def _teacher_forced(orc, prompt, gpu_tokens, embeds=None, pos=None, decode_pos=None):
    """Oracle logits for every step given the GPU's own token sequence; returns
    (argmax, top1-top2 margin, top1 - logit[gpu token]) per step."""
    st = orc.new_state()
    logits = orc.forward(st, prompt, embeds=embeds, position_ids=pos)
    out = []
    for i, tok in enumerate(gpu_tokens):
        ref = int(O.argmax_lowest(logits.unsqueeze(0))[0])
        top2 = torch.topk(logits.double(), 2).values
        out.append((ref, float(top2[0] - top2[1]), float(logits[ref] - logits[tok])))
        if i + 1 == len(gpu_tokens):
            break
        p = None if decode_pos is None else decode_pos(i)
        logits = orc.forward(st, torch.tensor([tok], dtype=torch.int32), position_ids=p)
    return out


@pytest.mark.parametrize("use_graph", [True, False])
def test_tiny_greedy_matches_oracle(gpu, use_graph):
    w = O.random_weights(_oracle_cfg(TINY), seed=11, std=0.2)
    prompt = torch.randint(0, TINY.vocab, (40,), generator=torch.Generator().manual_seed(3)).to(torch.int32)
    with tempfile.TemporaryDirectory() as tmp:
        eng, keep = _engine(tmp, TINY, w, max_tokens=128, max_new_tokens=24, use_graph=use_graph)
        req = edge_fm.Request(0, prompt.tolist())
        req.set_ignore_stop_tokens(True)
        toks = eng.generate(req).token_ids()
        m = eng.last_generate_metrics()
    assert len(toks) == 24 and m["decode_steps"] == 23
    orc = O.Qwen2Oracle(_oracle_cfg(TINY), O.fuse_weights(_oracle_cfg(TINY), w), max_tokens=128)
    exact = _check_against_oracle(toks, _teacher_forced(orc, prompt, toks), tol=0.05)
    assert exact >= 22


def test_graph_and_eager_agree_and_repeat(gpu):
    w = O.random_weights(_oracle_cfg(TINY), seed=12, std=0.2)
    prompt = list(range(5, 45))
    outs = []
    with tempfile.TemporaryDirectory() as tmp:
        for g in (True, False):
            eng, keep = _engine(tmp, TINY, w, max_tokens=128, max_new_tokens=30, use_graph=g)
            req = edge_fm.Request(0, prompt)
            req.set_ignore_stop_tokens(True)
            outs.append(eng.generate(req).token_ids())
            outs.append(eng.generate(req).token_ids())  # second call reuses the captured graph
            del eng
    assert outs[0] == outs[1] == outs[2] == outs[3]


def test_prefix_slot_and_stop_tokens_and_cap(gpu):
    w = O.random_weights(_oracle_cfg(TINY), seed=13, std=0.2)
    prompt = list(range(100, 150))
    with tempfile.TemporaryDirectory() as tmp:
        eng, keep = _engine(tmp, TINY, w, max_tokens=128, max_new_tokens=16)
        req = edge_fm.Request(0, prompt)
        req.set_ignore_stop_tokens(True)
        base = eng.generate(req).token_ids()
        del eng
        # fixed-prefix slot: the prefix is prefilled at warmup, generate prefills the suffix
        eng, keep = _engine(tmp, TINY, w, max_tokens=128, max_new_tokens=16, prefix_token_ids=prompt[:20])
        req = edge_fm.Request(0, prompt)
        req.set_ignore_stop_tokens(True)
        assert eng.generate(req).token_ids() == base
        # stop tokens truncate after the first hit, inclusive
        req2 = edge_fm.Request(0, prompt)
        req2.set_stop_token_ids([base[3]])
        got = eng.generate(req2).token_ids()
        assert got == base[: base.index(base[3]) + 1]
        del eng
        # generated-token cap: min(max_new_tokens, max_tokens - len + 1)
        eng, keep = _engine(tmp, TINY, w, max_tokens=55, max_new_tokens=16)
        req = edge_fm.Request(0, prompt)
        req.set_ignore_stop_tokens(True)
        got = eng.generate(req).token_ids()
        assert got == base[: 55 - 50 + 1]
        # invalid request id / empty request / out-of-vocab ids raise InvalidRequestError
        with pytest.raises(edge_fm.InvalidRequestError):
            eng.generate(edge_fm.Request(7, prompt))
        with pytest.raises(edge_fm.InvalidRequestError):
            eng.generate(edge_fm.Request(0, []))
        with pytest.raises(edge_fm.InvalidRequestError):
            eng.generate(edge_fm.Request(0, [1, 2, TINY.vocab]))


def test_prefix_restored_after_non_matching_request(gpu):
    """A request that does not start with the slot's prefix prefills over the prefix rows;
    the next request that does start with it must see the prefix again (it is re-prefilled),
    so its tokens equal a fresh engine's."""
    w = O.random_weights(_oracle_cfg(TINY), seed=14, std=0.2)
    prompt = list(range(200, 250))
    other = list(range(600, 640))
    with tempfile.TemporaryDirectory() as tmp:
        eng, keep = _engine(tmp, TINY, w, max_tokens=128, max_new_tokens=12, prefix_token_ids=prompt[:20])
        req = edge_fm.Request(0, prompt)
        req.set_ignore_stop_tokens(True)
        fresh = eng.generate(req).token_ids()
        req_o = edge_fm.Request(0, other)
        req_o.set_ignore_stop_tokens(True)
        other_toks = eng.generate(req_o).token_ids()
        again = eng.generate(req).token_ids()
        del eng
        eng, keep = _engine(tmp, TINY, w, max_tokens=128, max_new_tokens=12)
        plain = edge_fm.Request(0, other)
        plain.set_ignore_stop_tokens(True)
        assert eng.generate(plain).token_ids() == other_toks
    assert again == fresh


def test_tiny_vl_mrope_with_custom_embeddings(gpu):
    shape = TINY_VL
    cfg = _oracle_cfg(shape)
    w = O.random_weights(cfg, seed=14, std=0.2)
    n_vis, n_txt = 24, 8
    embed_token_id = 900
    ids = [embed_token_id + i for i in range(n_vis)] + list(range(10, 10 + n_txt))
    vis = (torch.randn(n_vis, shape.hidden, generator=torch.Generator().manual_seed(5))).to(torch.bfloat16)
    # (t, h, w) grid 1 x 4 x 6 for the vision rows, then text positions continue
    t = torch.zeros(n_vis, dtype=torch.int32)
    hh = torch.arange(n_vis, dtype=torch.int32) // 6
    ww = torch.arange(n_vis, dtype=torch.int32) % 6
    start = int(max(hh.max(), ww.max())) + 1
    txt = torch.arange(start, start + n_txt, dtype=torch.int32)
    pos = torch.stack([torch.cat([t, txt]), torch.cat([hh, txt]), torch.cat([ww, txt])]).contiguous()
    with tempfile.TemporaryDirectory() as tmp:
        eng, keep = _engine(tmp, shape, w, max_tokens=96, max_new_tokens=12, model_name="qwen2_5_vl")
        vis_g = vis.to("cuda:0")
        pos_g = pos.to("cuda:0")
        req = edge_fm.Request(0, ids, edge_fm.Tensor(vis_g.data_ptr(), list(vis_g.shape), edge_fm.DType.BFloat16,
                                                     edge_fm.Device.GPU, 0, False), embed_token_id,
                              edge_fm.Tensor(pos_g.data_ptr(), [3, len(ids)], edge_fm.DType.Int32,
                                             edge_fm.Device.GPU, 0, False))
        req.set_ignore_stop_tokens(True)
        toks = eng.generate(req).token_ids()
    assert len(toks) == 12
    orc = O.Qwen2Oracle(cfg, O.fuse_weights(cfg, w), max_tokens=96)
    emb = O.embedding(torch.tensor(ids, dtype=torch.int32), w["model.embed_tokens.weight"], vis, embed_token_id)
    last = int(pos.max())

    def dpos(i):  # decode step i+1 position: last + 1 + i (qwen2_5.cpp:932-955)
        return torch.full((3, 1), last + 1 + i, dtype=torch.int32)

    steps = _teacher_forced(orc, torch.tensor(ids, dtype=torch.int32), toks, embeds=emb, pos=pos, decode_pos=dpos)
    exact = _check_against_oracle(toks, steps, tol=0.05)
    assert exact >= 10


def test_qwen25_1p5b_shape_greedy_matches_oracle(gpu):
    """Full Qwen2.5-1.5B shape (28 layers, vocab 151936, tied head), random-init
    N(0, 0.02): 64-token prompt, 10 greedy tokens checked against the oracle."""
    shape = S.QWEN25_1P5B
    cfg = _oracle_cfg(shape)
    w = O.random_weights(cfg, seed=21, std=0.02)
    prompt = torch.randint(0, shape.vocab, (64,), generator=torch.Generator().manual_seed(4)).to(torch.int32)
    with tempfile.TemporaryDirectory() as tmp:
        eng, keep = _engine(tmp, shape, w, max_tokens=256, max_new_tokens=10)
        req = edge_fm.Request(0, prompt.tolist())
        req.set_ignore_stop_tokens(True)
        toks = eng.generate(req).token_ids()
        del eng, keep
    torch.cuda.empty_cache()
    orc = O.Qwen2Oracle(cfg, O.fuse_weights(cfg, w), max_tokens=256, cache_f32=True)
    steps = _teacher_forced(orc, prompt, toks)
    exact = _check_against_oracle(toks, steps, tol=0.05)
    # Every step whose oracle top-2 margin is >= 0.05 logits must match (the gap check
    # enforces it); with N(0, 0.02) weights the logits are nearly flat (spread ~0.8), so
    # near-ties below that margin may resolve either way under bf16 rounding.
    clear = sum(1 for _, margin, _ in steps if margin >= 0.05)
    assert clear >= 5 and exact >= clear


@pytest.mark.parametrize("use_graph", [True, False])
def test_tiny_top_p_sampling_matches_oracle(gpu, use_graph):
    """temperature 0.8 / top-p 0.9. The engine records every step's fp32 logits
    (runtime.debug_logits): every token must be exactly the oracle sampler's draw on the
    engine's own logits (same seed, draw counter = the token's response index), and those
    logits must follow the oracle's (teacher-forced on the GPU's tokens) within bf16
    noise. A wrong draw counter, a wrong logits buffer or a sampler change cannot hide."""
    T, P, SEED = 0.8, 0.9, 5
    w = O.random_weights(_oracle_cfg(TINY), seed=31, std=0.2)
    prompt = torch.randint(0, TINY.vocab, (32,), generator=torch.Generator().manual_seed(8)).to(torch.int32)
    with tempfile.TemporaryDirectory() as tmp:
        eng, keep = _engine(tmp, TINY, w, max_tokens=128, max_new_tokens=32, use_graph=use_graph, temperature=T,
                            top_p=P, seed=SEED, debug_logits=True)
        req = edge_fm.Request(0, prompt.tolist())
        req.set_ignore_stop_tokens(True)
        toks = eng.generate(req).token_ids()
        lg_gpu = eng.last_logits()
        again = eng.generate(req).token_ids()
        lg_again = eng.last_logits()
        del eng
    assert toks == again, "same seed must give the same tokens"
    assert (lg_gpu == lg_again).all(), "the same request must give the same logits bit for bit"
    assert len(toks) == 32 and lg_gpu.shape == (32, TINY.vocab)
    orc = O.Qwen2Oracle(_oracle_cfg(TINY), O.fuse_weights(_oracle_cfg(TINY), w), max_tokens=128)
    st = orc.new_state()
    logits = orc.forward(st, prompt)
    worst_max = worst_mean = 0.0
    for i, tok in enumerate(toks):
        ref, _ = O.sample_top_p(lg_gpu[i], T, P, SEED, i)
        assert tok == ref, f"step {i}: engine drew {tok}, the oracle sampler on the engine's logits draws {ref}"
        o = logits.numpy().astype(np.float64)
        d = np.abs(lg_gpu[i].astype(np.float64) - o)
        worst_max, worst_mean = max(worst_max, d.max() / o.std()), max(worst_mean, d.mean() / o.std())
        logits = orc.forward(st, torch.tensor([tok], dtype=torch.int32))
    print(f"tiny top-p: |logit - oracle| / logit std: max {worst_max:.4f}, mean {worst_mean:.5f}")
    # measured 0.435 / 0.081 (std-0.2 weights: larger activations, larger bf16 noise)
    assert worst_max < 0.65 and worst_mean < 0.12, f"engine logits off the oracle's: {worst_max:.4f} / {worst_mean:.5f}"


def test_prefill_split_k_scratch_is_shared_and_bounded(gpu):
    """Prefill at several prompt lengths on 1.5B-width layers (whose split-K GEMMs need
    scratch at these lengths): every projection takes its split-K scratch from one
    grow-only buffer per device, so its size only grows, ends at the largest single need of
    the lengths run (or what earlier work had already grown it to), and a second pass over
    the same lengths leaves it unchanged; the tokens do not depend on the order."""
    import efm_capi as C

    shape = S.ModelShape(hidden=1536, layers=2, heads=12, kv_heads=2, head_dim=128, inter=8960, vocab=1000)
    cfg = _oracle_cfg(shape)
    w = O.random_weights(cfg, seed=41, std=0.02)
    lib = C.load()
    H, I, qd, kvd = shape.hidden, shape.inter, shape.q_dim, shape.kv_dim
    lengths = [900, 300, 1200, 64, 700]
    need = max(max(lib.efm_linear_workspace_bytes(m, H, qd + 2 * kvd), lib.efm_linear_workspace_bytes(m, qd, H),
                   lib.efm_linear_workspace_bytes(m, I, H), lib.efm_fused_gate_up_swiglu_workspace_bytes(m, H, I))
               for m in lengths)
    assert need > 0, "these shapes must exercise the split-K scratch"
    before = edge_fm.linear_scratch_bytes(0)
    g = torch.Generator().manual_seed(9)
    prompts = {L: torch.randint(0, shape.vocab, (L,), generator=g).tolist() for L in lengths}
    sizes, toks = [], {}
    with tempfile.TemporaryDirectory() as tmp:
        eng, keep = _engine(tmp, shape, w, max_tokens=1300, max_new_tokens=2)
        for rep in range(2):
            for L in lengths:
                req = edge_fm.Request(0, prompts[L])
                req.set_ignore_stop_tokens(True)
                t = eng.generate(req).token_ids()
                if rep == 0:
                    toks[L] = t
                else:
                    assert t == toks[L], f"prompt {L}: tokens changed on the second pass"
                sizes.append(edge_fm.linear_scratch_bytes(0))
        del eng
    assert sizes == sorted(sizes), f"the scratch must only grow: {sizes}"
    assert sizes[-1] == max(before, need), f"scratch {sizes[-1]} bytes, largest need {need} (before {before})"
    assert sizes[len(lengths) - 1] == sizes[-1], "the second pass must not grow the scratch"


def test_top_p_sampling_seeds_differ_and_config_checks(gpu):
    w = O.random_weights(_oracle_cfg(TINY), seed=32, std=0.2)
    prompt = list(range(10, 40))
    outs = []
    with tempfile.TemporaryDirectory() as tmp:
        for seed in (1, 2):
            eng, keep = _engine(tmp, TINY, w, max_tokens=128, max_new_tokens=24, temperature=1.0, top_p=0.95,
                                seed=seed)
            req = edge_fm.Request(0, prompt)
            req.set_ignore_stop_tokens(True)
            outs.append(eng.generate(req).token_ids())
            del eng
        assert outs[0] != outs[1]
        mdir = S.write_model_dir(os.path.join(tmp, "model"), TINY)
        for bad in (dict(temperature=-0.5), dict(temperature=0.7, top_p=0.0)):
            ecfg = S.write_engine_config(os.path.join(tmp, "bad.json"), mdir, max_tokens=128, **bad)
            with pytest.raises(edge_fm.ConfigurationError):
                edge_fm.EdgeFM(ecfg)


TINY128 = S.ModelShape(hidden=256, layers=2, heads=2, kv_heads=1, head_dim=128, inter=512, vocab=1000)


@pytest.mark.parametrize("shape_id", ["tiny128", "1p5b"])
@pytest.mark.parametrize("use_graph", [True, False])
def test_head_dim_128_decode_matches_oracle(gpu, shape_id, use_graph):
    """Head-dim-128 text models (the engine's rotated-cache decode plan, graph-replayed or
    eager) against the oracle teacher-forced on the engine's own tokens: every flip is a
    near tie, every clear step matches, and a second generate() repeats the first bit for
    bit."""
    if shape_id == "tiny128":
        shape, seed, n_prompt, n_gen, std = TINY128, 41, 40, 24, 0.2
    else:
        shape, seed, n_prompt, n_gen, std = S.QWEN25_1P5B, 42, 64, 16, 0.02
    w = O.random_weights(_oracle_cfg(shape), seed=seed, std=std)
    prompt = torch.randint(0, shape.vocab, (n_prompt,), generator=torch.Generator().manual_seed(6)).to(torch.int32)
    orc = O.Qwen2Oracle(_oracle_cfg(shape), O.fuse_weights(_oracle_cfg(shape), w), max_tokens=256,
                        cache_f32=shape_id != "tiny128")
    with tempfile.TemporaryDirectory() as tmp:
        eng, keep = _engine(tmp, shape, w, max_tokens=256, max_new_tokens=n_gen, use_graph=use_graph)
        req = edge_fm.Request(0, prompt.tolist())
        req.set_ignore_stop_tokens(True)
        first = eng.generate(req).token_ids()
        assert eng.generate(req).token_ids() == first, "rerun differs"
        del eng, keep
    steps = _teacher_forced(orc, prompt, first)
    _check_against_oracle(first, steps, tol=0.05)   # every flip is a near tie
    clear = [(tok, ref) for tok, (ref, margin, _) in zip(first, steps) if margin >= 0.05]
    assert all(tok == ref for tok, ref in clear), "a clear step differs"
    assert len(clear) >= 4, f"only {len(clear)} clear steps"


def test_compact_vocab_generate_matches_unmapped_run(gpu):
    """A pre-pruned checkpoint (vocab 600 of an original 1000, non-monotonic id map) run
    with compact_vocab enabled takes and returns original ids: its tokens are the
    unmapped run's tokens mapped through new_to_old, also with a remapped fixed KV
    prefix; request stop ids are remapped and pruned request ids are rejected
    (standard_engine.cpp:877-917,1070-1072; kv_manager.cpp:151-155)."""
    shape = S.ModelShape(hidden=256, layers=2, heads=4, kv_heads=2, head_dim=64, inter=512, vocab=600)
    w = O.random_weights(_oracle_cfg(shape), seed=31, std=0.2)
    g = torch.Generator().manual_seed(8)
    new_to_old = torch.randperm(1000, generator=g)[:600].tolist()
    prompt = torch.randint(0, 600, (40,), generator=g).tolist()
    external = [new_to_old[t] for t in prompt]
    with tempfile.TemporaryDirectory() as tmp:
        eng, keep = _engine(tmp, shape, w, max_tokens=96, max_new_tokens=20)
        req = edge_fm.Request(0, prompt)
        req.set_ignore_stop_tokens(True)
        base = eng.generate(req).token_ids()
        del eng
        S.write_compact_vocab_mapping(os.path.join(tmp, "compact_vocab.json"), 1000, new_to_old, [new_to_old[0]])
        cv = {"enabled": True, "mapping_path": "compact_vocab.json", "reject_unknown_input_ids": True}
        eng, keep = _engine(tmp, shape, w, max_tokens=96, max_new_tokens=20, compact_vocab=cv,
                            prefix_token_ids=external[:12])
        req = edge_fm.Request(0, external)
        req.set_ignore_stop_tokens(True)
        got = eng.generate(req).token_ids()
        assert got == [new_to_old[t] for t in base]
        assert eng.last_generate_metrics()["prefill_tokens"] == 40 - 12
        req2 = edge_fm.Request(0, external)
        req2.set_stop_token_ids([got[4]])
        assert eng.generate(req2).token_ids() == got[: got.index(got[4]) + 1]
        pruned = sorted(set(range(1000)) - set(new_to_old))[0]
        with pytest.raises(edge_fm.InvalidRequestError):
            eng.generate(edge_fm.Request(0, external[:5] + [pruned]))
        del eng


@pytest.mark.parametrize("table", ["generic", "fused", "split_o1_plain"])
def test_decode_impls_switched_by_table_match_oracle(gpu, knob, table):
    """Operator-table records switch the decode attention impl (all layers) or one layer's
    o_proj; every variant generates the oracle's tokens (teacher-forced, near-tie rule)
    and agrees with the default plan's run at every clear step. The fused launch writes
    128-key split partials, so its run keeps the partials plan off one-tile splits (which
    a 128-row bound would otherwise take) with EFM_KNOB_DECODE_TILE."""
    import json
    import efm_capi as C

    fused = "hip_gfx950_decode_fused_qkv_attention"
    recs = {"generic": [{"op_kind": "attention", "stage": "decode", "impl_id": "hip_gfx950_attention"}],
            "fused": [{"op_kind": "attention", "stage": "decode", "impl_id": fused}],
            "split_o1_plain": [{"op_kind": "linear", "op_name": "model.layers.1.self_attn.o_proj", "stage": "decode",
                                "impl_id": "hip_gfx950_linear"}]}[table]
    shape = TINY128
    w = O.random_weights(_oracle_cfg(shape), seed=43, std=0.2)
    prompt = torch.randint(0, shape.vocab, (40,), generator=torch.Generator().manual_seed(9)).to(torch.int32)
    with tempfile.TemporaryDirectory() as tmp:
        path = os.path.join(tmp, "table.json")
        with open(path, "w") as f:
            json.dump({"schema": "edgefm_operator_impl_table_v1", "records": recs}, f)
        runs = {}
        for name, tpath in (("default", ""), (table, path)):
            knob(C.EFM_KNOB_DECODE_TILE, 1 if name == "fused" else 0)
            eng, keep = _engine(tmp, shape, w, max_tokens=96, max_new_tokens=24, operator_impl_table_path=tpath)
            plan = edge_fm.plan_decode(os.path.join(tmp, "engine.json"), 96)
            req = edge_fm.Request(0, prompt.tolist())
            req.set_ignore_stop_tokens(True)
            runs[name] = (eng.generate(req).token_ids(), plan)
            del eng
    plan = runs[table][1]
    want = {"generic": "hip_gfx950_attention", "fused": fused}.get(
        table, "hip_gfx950_decode_split_attention")
    assert all(p["attention"] == want for p in plan)
    assert all(p["attention"] == "hip_gfx950_decode_split_attention" for p in runs["default"][1])
    if table == "split_o1_plain":
        assert plan[0]["partials_to_o_proj"] and not plan[1]["partials_to_o_proj"]
    orc = O.Qwen2Oracle(_oracle_cfg(shape), O.fuse_weights(_oracle_cfg(shape), w), max_tokens=96)
    for name, (toks, _) in runs.items():
        steps = _teacher_forced(orc, prompt, toks)
        exact = _check_against_oracle(toks, steps, tol=0.05)
        assert exact >= 20, f"{name}: {exact}/24 exact"



@pytest.mark.parametrize("use_graph", [False, True])
def test_front_wait_timeout_raises_device_error_then_recovers(gpu, knob, use_graph):
    """The fused front half (selected by a table record)'s bounded wait forced to give up from the host
    (EFM_KNOB_FRONT_WAIT_TIMEOUT: its attention splits wait for a tag that no word
    carries, 64 polls; every kernel still drains): generate() raises DeviceError and
    returns no tokens. With the knob back at 0 the same engine's next generate() returns
    the tokens of an engine that never failed (after the error the engine drops its
    captured decode graphs, so the graph case captures the next call afresh). The fused
    launch writes 128-key split partials: EFM_KNOB_DECODE_TILE keeps the partials plan of
    the short bounds on them."""
    import json
    import efm_capi as C

    shape = TINY128
    w = O.random_weights(_oracle_cfg(shape), seed=44, std=0.2)
    prompt = torch.randint(0, shape.vocab, (40,), generator=torch.Generator().manual_seed(10)).tolist()
    with tempfile.TemporaryDirectory() as tmp:
        table = os.path.join(tmp, "table.json")
        with open(table, "w") as f:
            json.dump({"schema": "edgefm_operator_impl_table_v1",
                       "records": [{"op_kind": "attention", "stage": "decode",
                                    "impl_id": "hip_gfx950_decode_fused_qkv_attention"}]}, f)
        knob(C.EFM_KNOB_DECODE_TILE, 1)
        cfg = dict(max_tokens=96, max_new_tokens=16, use_graph=use_graph, operator_impl_table_path=table)
        eng, keep = _engine(tmp, shape, w, **cfg)
        plan = edge_fm.plan_decode(os.path.join(tmp, "engine.json"), 96)
        assert all(p["attention"] == "hip_gfx950_decode_fused_qkv_attention" for p in plan)
        req = edge_fm.Request(0, prompt)
        req.set_ignore_stop_tokens(True)
        clean = eng.generate(req).token_ids()
        del eng
        eng, keep = _engine(tmp, shape, w, **cfg)
        knob(C.EFM_KNOB_FRONT_WAIT_TIMEOUT, 1)
        with pytest.raises(edge_fm.DeviceError, match="timed out"):
            eng.generate(req)
        knob(C.EFM_KNOB_FRONT_WAIT_TIMEOUT, 0)
        assert eng.generate(req).token_ids() == clean
        assert eng.generate(req).token_ids() == clean
        del eng
