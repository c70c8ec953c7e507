"""End-to-end GPU parity at the BASELINE configurations' own shapes: the C++ engine
(`edge_fm.EdgeFM.generate`, HIP graphs on) against the CPU oracle, teacher-forced on the
GPU's tokens.

  * C2 (the headline): the full Qwen2.5-1.5B shape, N(0, 0.02) weights as in bench.py, a
    512-token uniform-random prompt, 32 greedy tokens.
  * C5's model: the full Qwen2.5-7B shape with its untied LM head (lm_head.weight apart
    from the embedding table), a short prompt, temperature 0.7 / top-p 0.9 sampling.
  * C3's model: the full Qwen2.5-VL-3B shape, 1280 N(0, 1) vision rows on a 1 x 32 x 40
    (t, h, w) grid with 3-D M-RoPE positions plus 64 text tokens, a short greedy decode
    from position last + 1.

The engine records every step's fp32 logits (runtime.debug_logits). Each token must be
exactly the argmax (greedy) or the oracle sampler's draw (top-p: same seed, draw counter =
response index) on the engine's own logits; the production configuration (fused LM-head
top-1 for greedy) must give the same tokens; a rerun must repeat tokens and logits bit for
bit; the engine's logits must follow the oracle's, teacher-forced on the GPU's tokens,
within stated bounds (in units of the step's logit std); and greedy steps whose oracle
top-2 margin lies far outside that noise must give the oracle's token. Each test prints
its per-step figures.

Weights are generated on the GPU from a seed (S.synthetic_weights_gpu: N(0, std), norm
weights ones) and copied to the host for the oracle. Mirrors
tests/engine/test_qwen2_generate.py:758-788,1021-1237 of the reference (its HF dumps are
replaced by the oracle, which tests/test_oracle.py pins to the HF model)."""
import os
import tempfile
import time

import numpy as np
import pytest
import torch

import edge_fm
import efm_setup as S
from oracle import efm_oracle as O

pytestmark = pytest.mark.gpu

# Accepted |engine logit - oracle logit| in units of the step's logit std: (max over the
# vocabulary, mean over the vocabulary); for greedy configs also the oracle top-2 margin
# (in logit stds) above which the token must be the oracle's, and how many such steps the
# run must hold. Measured on MI355X (max / mean): C2 0.169 / 0.029, 7B 0.294 / 0.043,
# VL-3B 0.255 / 0.044. The bounds sit about 1.5x above; an error in any operator moves
# the mean by an order of magnitude. The clear-step margin is >= 5 standard deviations
# of the noise on the difference of two logits (about 1.8 x the mean error): below it a
# flip is bf16 noise. On the VL-3B shape that noise is the model's own: nudging 1 % of
# the oracle's attention outputs by one bf16 ulp moves its logits by up to 0.2 (0.03 on
# average), as much as the whole engine-oracle difference.
C2_TOL = (0.3, 0.05, 0.3, 4)
B7_TOL = (0.45, 0.07)
VL_TOL = (0.4, 0.07, 0.45, 0)


def _cfg(shape):
    return O.QwenConfig(hidden=shape.hidden, layers=shape.layers, heads=shape.heads, kv_heads=shape.kv_heads,
                        head_dim=shape.head_dim, inter=shape.inter, vocab=shape.vocab, eps=shape.eps,
                        theta=shape.theta, tied=shape.tied, mrope_section=shape.mrope_section)


def _log(msg):
    print(f"[e2e {time.strftime('%H:%M:%S')}] {msg}", flush=True)


def _oracle_from_gpu(shape, wdev, max_tokens):
    """Oracle over host copies of the engine's own device weights (fp32 weight cache)."""
    cfg = _cfg(shape)
    wcpu = {k: v.cpu() for k, v in wdev.items()}
    orc = O.Qwen2Oracle(cfg, O.fuse_weights(cfg, wcpu), max_tokens=max_tokens, cache_f32=True)
    del wcpu
    return orc


def _run_engine(tmp, shape, wdev, req, **cfg):
    """Runs the request on an engine that records every step's fp32 logits
    (runtime.debug_logits) twice (tokens and logits must repeat bit for bit), then once
    on the production configuration (greedy: the fused LM-head top-1), whose tokens must
    be the same. Returns (tokens, logits [steps, vocab])."""
    S.register_weights(wdev)
    mdir = S.write_model_dir(os.path.join(tmp, "model"), shape)
    req.set_ignore_stop_tokens(True)
    ecfg = S.write_engine_config(os.path.join(tmp, "engine_dbg.json"), mdir, debug_logits=True, **cfg)
    eng = edge_fm.EdgeFM(ecfg)
    toks = eng.generate(req).token_ids()
    lg = eng.last_logits()
    again = eng.generate(req).token_ids()
    lg_again = eng.last_logits()
    del eng
    assert toks == again, "the same request must give the same tokens"
    assert (lg == lg_again).all(), "the same request must give the same logits bit for bit"
    ecfg = S.write_engine_config(os.path.join(tmp, "engine.json"), mdir, **cfg)
    eng = edge_fm.EdgeFM(ecfg)
    prod = eng.generate(req).token_ids()
    del eng
    torch.cuda.synchronize()
    assert prod == toks, "the production configuration (fused LM-head top-1) must give the recorded tokens"
    return toks, lg


def _oracle_logits(orc, prompt, toks, embeds=None, pos=None, decode_pos=None):
    """The oracle's fp32 logits for every step, teacher-forced on the GPU's tokens."""
    st = orc.new_state()
    logits = orc.forward(st, prompt, embeds=embeds, position_ids=pos)
    out = []
    for i, tok in enumerate(toks):
        out.append(logits.numpy().astype(np.float32))
        if i + 1 < len(toks):
            p = None if decode_pos is None else decode_pos(i)
            logits = orc.forward(st, torch.tensor([tok], dtype=torch.int32), position_ids=p)
    return np.stack(out)


def _logit_errors(tag, lg_gpu, lg_orc):
    """Per step: max and mean |engine logit - oracle logit| relative to the spread (std)
    of the oracle's logits of that step."""
    out = []
    for g, o in zip(lg_gpu, lg_orc):
        d = np.abs(g.astype(np.float64) - o.astype(np.float64))
        sd = float(o.astype(np.float64).std())
        out.append((float(d.max()) / sd, float(d.mean()) / sd, float(d.max()), float(d.mean())))
    _log(f"{tag}: |logit - oracle| / logit std per step: max {max(e[0] for e in out):.4f}, "
         f"mean {max(e[1] for e in out):.5f} (absolute: max {max(e[2] for e in out):.4f}, "
         f"mean {np.mean([e[3] for e in out]):.5f})")
    return out


def _check_logits(tag, errs, tol_max, tol_mean):
    worst_max, worst_mean = max(e[0] for e in errs), max(e[1] for e in errs)
    assert worst_mean <= tol_mean, f"{tag}: mean logit error {worst_mean:.5f} logit std (> {tol_mean})"
    assert worst_max <= tol_max, f"{tag}: max logit error {worst_max:.4f} logit std (> {tol_max})"


def _check_greedy(tag, toks, lg_gpu, lg_orc, tol_max, tol_mean, clear_sd, min_clear):
    """Every token is the argmax (lowest index on ties) of the engine's own logits; the
    engine's logits follow the oracle's (errors in units of the step's logit std, bounded
    by tol_max / tol_mean); and wherever the oracle's top-2 margin exceeds clear_sd logit
    stds the token is the oracle's argmax."""
    errs = _logit_errors(tag, lg_gpu, lg_orc)
    report, clear = [], 0
    for i, tok in enumerate(toks):
        g, o = lg_gpu[i], lg_orc[i]
        assert tok == int(O.argmax_lowest(torch.from_numpy(g).unsqueeze(0))[0]), \
            f"{tag} step {i}: token {tok} is not the argmax of the engine's logits"
        ref = int(O.argmax_lowest(torch.from_numpy(o).unsqueeze(0))[0])
        top2 = np.sort(o.astype(np.float64))[-2:]
        margin = float(top2[1] - top2[0]) / float(o.astype(np.float64).std())
        report.append(f"{tok}/{ref}/{margin:.3f}/{errs[i][0]:.3f}")
        if margin > clear_sd:
            clear += 1
            assert tok == ref, f"{tag} step {i}: clear step (oracle margin {margin:.4f} std) gives {tok}, oracle {ref}"
    _log(f"{tag} per-step (gpu, oracle, oracle top-2 margin / std, max |logit - oracle| / std): " + " ".join(report))
    _log(f"{tag}: {clear} clear steps (margin > {clear_sd} std) all match")
    _check_logits(tag, errs, tol_max, tol_mean)
    assert clear >= min_clear, f"{tag}: only {clear} steps with a clear oracle margin"


def test_c2_headline_512_prompt_32_greedy_tokens(gpu):
    shape = S.QWEN25_1P5B
    P, G = 512, 32
    _log("C2: generating weights")
    wdev = S.synthetic_weights_gpu(shape, seed=3, std=0.02)
    prompt = torch.randint(0, shape.vocab, (P,), generator=torch.Generator().manual_seed(11)).to(torch.int32)
    with tempfile.TemporaryDirectory() as tmp:
        toks, lg = _run_engine(tmp, shape, wdev, edge_fm.Request(0, prompt.tolist()), max_tokens=P + G,
                               max_new_tokens=G, use_graph=True)
    assert len(toks) == G
    _log("C2: oracle")
    orc = _oracle_from_gpu(shape, wdev, P + G)
    del wdev
    torch.cuda.empty_cache()
    _check_greedy("C2 1.5B 512+32", toks, lg, _oracle_logits(orc, prompt, toks), *C2_TOL)


def test_7b_shape_untied_head_top_p_sampling(gpu):
    """All 28 layers of the 7B shape with an untied LM head. The head is drawn with std
    0.08 (logit spread ~5) so that the top-p 0.9 nucleus at T = 0.7 holds tens of tokens
    and the sampler's choice is a real test; with std 0.02 the nucleus would be most of
    the 152064-token vocabulary and every draw would sit within noise of a boundary."""
    shape = S.QWEN25_7B
    assert not shape.tied
    P, G, T, TOP_P, SEED = 16, 16, 0.7, 0.9, 1234
    _log("7B: generating weights")
    wdev = S.synthetic_weights_gpu(shape, seed=5, std=0.02)
    g = torch.Generator(device="cuda:0").manual_seed(6)
    wdev["lm_head.weight"] = (torch.randn(shape.vocab, shape.hidden, device="cuda:0", generator=g) * 0.08).to(
        torch.bfloat16)
    prompt = torch.randint(0, shape.vocab, (P,), generator=torch.Generator().manual_seed(12)).to(torch.int32)
    with tempfile.TemporaryDirectory() as tmp:
        toks, lg = _run_engine(tmp, shape, wdev, edge_fm.Request(0, prompt.tolist()), max_tokens=P + G,
                               max_new_tokens=G, use_graph=True, temperature=T, top_p=TOP_P, seed=SEED)
    assert len(toks) == G
    _log("7B: oracle")
    orc = _oracle_from_gpu(shape, wdev, P + G)
    del wdev
    torch.cuda.empty_cache()
    lg_orc = _oracle_logits(orc, prompt, toks)
    errs = _logit_errors("7B", lg, lg_orc)
    report, nuclei = [], []
    for i, tok in enumerate(toks):
        # the draw: exactly the oracle sampler's on the engine's own logits (same seed,
        # counter = response index), with no allowance
        ref, info = O.sample_top_p(lg[i], T, TOP_P, SEED, i)
        assert tok == ref, f"7B step {i}: engine drew {tok}, the oracle sampler on the engine's logits draws {ref}"
        nuclei.append(info["nucleus"])
        report.append(f"{tok}/{info['nucleus']}/{errs[i][0]:.3f}")
    _log("7B per-step (token, nucleus size, max |logit - oracle| / std): " + " ".join(report))
    assert max(nuclei) > 1, "nucleus never held more than one token: the test would not exercise sampling"
    _check_logits("7B", errs, *B7_TOL)


def test_vl3b_shape_1280_vision_rows_mrope(gpu):
    """All 36 layers of the VL-3B shape, M-RoPE sections 16/24/24; the vision rows sit on
    the (t, h, w) grid (0, r // 40, r % 40), the text rows at 40 + j on all three axes, and
    decode step i at last + 1 + i with last = the largest prompt position. Weights
    N(0, 0.02) as in bench.py (tied head)."""
    shape = S.QWEN25_VL_3B
    nv, nt, G = 1280, 64, 16
    _log("VL-3B: generating weights")
    wdev = S.synthetic_weights_gpu(shape, seed=7, std=0.02)
    g = torch.Generator().manual_seed(13)
    embed_id = shape.vocab + 1000
    text = torch.randint(0, shape.vocab, (nt,), generator=g).tolist()
    ids = [embed_id + i for i in range(nv)] + text
    vis = torch.randn(nv, shape.hidden, generator=g).to(torch.bfloat16)
    pos = torch.empty(3, nv + nt, dtype=torch.int32)
    r = torch.arange(nv)
    pos[0, :nv] = 0
    pos[1, :nv] = r // 40
    pos[2, :nv] = r % 40
    pos[:, nv:] = (40 + torch.arange(nt)).to(torch.int32)
    last = int(pos.max())
    vis_g, pos_g = vis.to("cuda:0"), pos.to("cuda:0")
    req = edge_fm.Request(0, ids, edge_fm.Tensor(vis_g.data_ptr(), list(vis_g.shape), edge_fm.DType.BFloat16,
                                                 edge_fm.Device.GPU, 0, False), embed_id,
                          edge_fm.Tensor(pos_g.data_ptr(), [3, len(ids)], edge_fm.DType.Int32, edge_fm.Device.GPU, 0,
                                         False))
    with tempfile.TemporaryDirectory() as tmp:
        toks, lg = _run_engine(tmp, shape, wdev, req, max_tokens=nv + nt + G, max_new_tokens=G, use_graph=True,
                               model_name="qwen2_5_vl")
    assert len(toks) == G
    _log("VL-3B: oracle")
    orc = _oracle_from_gpu(shape, wdev, nv + nt + G)
    emb = O.embedding(torch.tensor(ids, dtype=torch.int32), orc.w["embed"].to(torch.bfloat16), vis, embed_id)
    del wdev
    torch.cuda.empty_cache()

    def dpos(i):
        return torch.full((3, 1), last + 1 + i, dtype=torch.int32)

    lg_orc = _oracle_logits(orc, torch.tensor(ids, dtype=torch.int32), toks, embeds=emb, pos=pos, decode_pos=dpos)
    _check_greedy("VL-3B 1280 vision + 64 text", toks, lg, lg_orc, *VL_TOL)
