"""GPU parity of the temperature / top-p sampler (efm_sampler_top_p) with the oracle's
exact integer-mass definition. Tokens must be identical; the only allowed difference
is a decision whose boundary lies within 1e-5 (relative) of the random target, where a
one-ulp difference between the device's and the host's expf may move it. Edge cases
follow the reference's sampler tests (tests/layers/test_sampler.py): tiny and
vocab-sized rows, a dominant logit, ties, temperatures far from 1."""
import numpy as np
import pytest
import torch

import efm_capi as C
from oracle import efm_oracle as O
from _util import ptr, stream

pytestmark = pytest.mark.gpu

MARGIN = 1e-5


def _ws(gpu, vocab):
    # garbage-filled on purpose: the sampler needs no initial workspace contents
    n = C.load().efm_sampler_top_p_workspace_bytes(vocab)
    return torch.full((n,), 0xA5, dtype=torch.uint8, device=gpu)


def _gpu_sample(gpu, logits, T, p, seed, offset, d_offset=None):
    lg = torch.from_numpy(np.ascontiguousarray(logits, dtype=np.float32)).to(gpu)
    out = torch.full((1,), -1, dtype=torch.int32, device=gpu)
    ws = _ws(gpu, lg.numel())
    C.call("efm_sampler_top_p", lg.numel(), ptr(lg), float(T), float(p), seed, offset, ptr(d_offset), ptr(out),
           ptr(ws), ws.numel(), stream())
    torch.cuda.synchronize()
    return int(out.item())


def _check(gpu, logits, T, p, seed, offset):
    want, info = O.sample_top_p(logits, T, p, seed, offset)
    got = _gpu_sample(gpu, logits, T, p, seed, offset)
    if got != want:
        margin = O.sample_margin(logits, T, p, seed, offset)
        assert margin < MARGIN, f"token {got} != {want} (T={T} p={p} seed={seed} off={offset} margin={margin:.3g})"
    return got, want, info


@pytest.mark.parametrize("vocab", [1, 2, 7, 1000, 32000, 151936, 152064])
@pytest.mark.parametrize("T,p", [(0.7, 0.9), (1.0, 1.0), (0.3, 0.5), (2.0, 0.99)])
def test_sampler_top_p_matches_oracle(gpu, vocab, T, p):
    rng = np.random.default_rng(vocab)
    logits = (rng.standard_normal(vocab) * 4).astype(np.float32)
    exact = 0
    for off in range(6):
        got, want, _ = _check(gpu, logits, T, p, seed=20240601, offset=off)
        exact += got == want
    assert exact >= 5


def test_sampler_top_p_llm_like_logits(gpu):
    """Peaked logits like an LM head's: a few large values over a wide tail."""
    rng = np.random.default_rng(5)
    logits = (rng.standard_normal(151936) * 2).astype(np.float32)
    logits[rng.integers(0, 151936, 20)] += rng.uniform(8, 14, 20).astype(np.float32)
    for off in range(16):
        _check(gpu, logits, 0.7, 0.9, seed=42, offset=off)


def test_sampler_top_p_flat_logits_large_nucleus(gpu):
    """Nearly uniform logits (a random-init LM head): the nucleus holds ~90 % of the
    vocabulary, so the located token can sit in any of the 149 logit blocks."""
    rng = np.random.default_rng(8)
    logits = (rng.standard_normal(152064) * 0.05).astype(np.float32)
    seen = set()
    for off in range(24):
        got, want, info = _check(gpu, logits, 0.7, 0.9, seed=1234, offset=off)
        assert info["nucleus"] > 100000
        seen.add(got // 1024)
    assert len(seen) > 12


def test_sampler_top_p_workspace_reuse(gpu):
    """One workspace across calls of different vocabulary sizes and top-p modes."""
    ws = _ws(gpu, 152064)
    rng = np.random.default_rng(21)
    for i, (V, p) in enumerate([(152064, 0.9), (1000, 1.0), (32000, 0.5), (7, 0.9), (151936, 1.0)]):
        logits = (rng.standard_normal(V) * 3).astype(np.float32)
        lg = torch.from_numpy(logits).to(gpu)
        out = torch.full((1,), -1, dtype=torch.int32, device=gpu)
        C.call("efm_sampler_top_p", V, ptr(lg), 0.8, p, 99, i, None, ptr(out), ptr(ws), ws.numel(), stream())
        torch.cuda.synchronize()
        want, _ = O.sample_top_p(logits, 0.8, p, 99, i)
        got = int(out.item())
        assert got == want or O.sample_margin(logits, 0.8, p, 99, i) < MARGIN, (V, p)


def test_sampler_top_p_ties_and_dominant(gpu):
    # a dominant logit with T small: always the maximum
    logits = np.zeros(50000, dtype=np.float32)
    logits[31337] = 60.0
    for off in range(4):
        assert _gpu_sample(gpu, logits, 0.5, 0.9, 1, off) == 31337
    # exact ties: equal logits -> uniform over them; boundary ties all kept
    logits = np.full(4096, -20.0, dtype=np.float32)
    logits[[3, 100, 4000]] = 2.0
    seen = set()
    for off in range(64):
        got, want, info = _check(gpu, logits, 1.0, 0.5, 9, off)
        assert info["nucleus"] == 3
        seen.add(got)
    assert seen == {3, 100, 4000}


def test_sampler_top_p_device_offset_and_seed_words(gpu):
    rng = np.random.default_rng(11)
    logits = rng.standard_normal(32000).astype(np.float32)
    d_off = torch.tensor([17], dtype=torch.int32, device=gpu)
    a = _gpu_sample(gpu, logits, 1.0, 0.95, (3 << 40) | 5, 100, d_offset=d_off)
    want, _ = O.sample_top_p(logits, 1.0, 0.95, (3 << 40) | 5, 117)
    assert a == want or O.sample_margin(logits, 1.0, 0.95, (3 << 40) | 5, 117) < MARGIN


def test_sampler_top_p_deterministic(gpu):
    rng = np.random.default_rng(3)
    logits = rng.standard_normal(151936).astype(np.float32) * 3
    toks = {_gpu_sample(gpu, logits, 0.8, 0.9, 77, 5) for _ in range(8)}
    assert len(toks) == 1


def test_sampler_top_p_distribution(gpu):
    """Over many offsets the device's draws follow softmax(l / T) on the nucleus."""
    from scipy.stats import chisquare
    logits = np.array([2.0, 1.5, 1.0, 0.4, 0.0, -0.5, -1.0, -3.0], dtype=np.float32)
    T = 0.9
    pr = np.exp((logits.astype(np.float64) - logits.max()) / T)
    pr /= pr.sum()
    lg = torch.from_numpy(logits).to(gpu)
    n = 4000
    outs = torch.empty(n, dtype=torch.int32, device=gpu)
    ws = _ws(gpu, 8)
    for off in range(n):
        C.call("efm_sampler_top_p", 8, ptr(lg), T, 1.0, 2024, off, None, outs.data_ptr() + 4 * off, ptr(ws),
               ws.numel(), stream())
    torch.cuda.synchronize()
    counts = np.bincount(outs.cpu().numpy(), minlength=8)
    assert chisquare(counts, pr * n).pvalue > 1e-4


@pytest.mark.parametrize("bad", ["vocab0", "vocab_big", "temp0", "temp_nan", "top_p0", "small_ws"])
def test_sampler_top_p_rejects_bad_arguments(gpu, bad):
    lg = torch.zeros(16, dtype=torch.float32, device=gpu)
    out = torch.zeros(1, dtype=torch.int32, device=gpu)
    args = dict(vocab=16, T=1.0, p=0.9)
    if bad == "vocab0":
        args["vocab"] = 0
    elif bad == "vocab_big":
        args["vocab"] = (1 << 20) + 1
    elif bad == "temp0":
        args["T"] = 0.0
    elif bad == "temp_nan":
        args["T"] = float("nan")
    elif bad == "top_p0":
        args["p"] = 0.0
    ws = _ws(gpu, 16)
    if bad == "small_ws":
        ws = ws[:64]
    with pytest.raises(C.EfmError):
        C.call("efm_sampler_top_p", args["vocab"], ptr(lg), args["T"], args["p"], 1, 0, None, ptr(out), ptr(ws),
               ws.numel(), stream())
