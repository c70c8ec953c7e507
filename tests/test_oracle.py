"""CPU tests that pin the oracle (oracle/efm_oracle.py) before it is trusted.

The reference ships no golden vectors (its end-to-end oracle is HF transformers run
on downloaded checkpoints, tests/engine/test_qwen2_generate.py:199-284), so every
oracle function is pinned here by something other than its own formula:
closed forms evaluated independently in float64 numpy, library routines (HF
transformers' Qwen2 rotary embedding, Qwen2.5-VL multimodal rotary embedding and the
whole Qwen2ForCausalLM, torch's scaled_dot_product_attention, scipy's expit),
brute force on tiny inputs, and invariants (relative-position property of RoPE,
split-KV merge == unsplit softmax). Each check is chosen so that a plausible
mistake (wrong pairing, sign, section, dropped bias, residual rounded at the wrong
point, transposed weight, off-by-one position) fails it."""
import math

import numpy as np
import pytest
import torch

from oracle import efm_oracle as O

torch.manual_seed(0)


def _np(x):
    return x.detach().to(torch.float64).numpy()


# ----------------------------------------------------------------------------------
def test_rms_norm_closed_form():
    x = torch.randn(3, 1536).to(torch.bfloat16)
    w = (1 + 0.1 * torch.randn(1536)).to(torch.bfloat16)
    xs = _np(x)
    ref = xs / np.sqrt((xs ** 2).mean(-1, keepdims=True) + 1e-6) * _np(w)
    got = _np(O.rms_norm(x, w, 1e-6))
    assert np.max(np.abs(got - ref) / (np.abs(ref) + 1e-3)) < 2 ** -8  # within one bf16 rounding
    # scale invariance of RMSNorm (kills "sum instead of mean" and eps-outside-sqrt slips)
    assert torch.equal(O.rms_norm(x * 4, w, 0.0), O.rms_norm(x, w, 0.0))


def test_fused_add_rms_norm_rounding_points():
    """residual <- bf16(x + r) and the normalisation uses the fp32 sum
    (tests/operators/test_norm_sampler.py:82-86)."""
    x = torch.randn(2, 896).to(torch.bfloat16)
    r = torch.randn(2, 896).to(torch.bfloat16)
    w = torch.ones(896, dtype=torch.bfloat16)
    out, res = O.fused_add_rms_norm(x, r, w, 1e-6)
    s = _np(x) + _np(r)
    assert np.array_equal(_np(res), _np(torch.from_numpy(s).to(torch.float32).to(torch.bfloat16)))
    ref = s / np.sqrt((s ** 2).mean(-1, keepdims=True) + 1e-6)
    assert np.max(np.abs(_np(out) - ref)) < 2e-2


def test_linear_closed_form_and_layout():
    x = torch.randn(5, 64).to(torch.bfloat16)
    w = torch.randn(48, 64).to(torch.bfloat16)
    b = torch.randn(48).to(torch.bfloat16)
    ref = _np(x) @ _np(w).T + _np(b)
    assert np.allclose(_np(O.linear(x, w, b, out_f32=True)), ref, rtol=1e-5, atol=1e-4)
    assert np.allclose(_np(O.linear(x, w, b)), ref, rtol=2 ** -7, atol=1e-2)


def test_silu_and_layouts():
    from scipy.special import expit

    x = (torch.randn(3, 2 * 40) * 4).to(torch.bfloat16)
    up, gate = _np(x)[:, :40], _np(x)[:, 40:]
    ref = gate * expit(gate) * up
    assert np.allclose(_np(O.act_and_mul(x, up_first=True)), ref, rtol=1e-2, atol=1e-2)
    ref2 = up * expit(up) * gate  # [gate | up] layout swaps the roles
    assert np.allclose(_np(O.act_and_mul(x, up_first=False)), ref2, rtol=1e-2, atol=1e-2)


# ----------------------------------------------------------------------------------
def _hf_rotary(hd, theta, positions):
    from transformers import Qwen2Config
    from transformers.models.qwen2 import modeling_qwen2 as m

    cfg = Qwen2Config(hidden_size=hd * 2, num_attention_heads=2, num_key_value_heads=1, head_dim=hd,
                      rope_parameters={"rope_type": "default", "rope_theta": theta})
    rot = m.Qwen2RotaryEmbedding(cfg)
    dummy = torch.zeros(1, dtype=torch.float32)
    cos, sin = rot(dummy, positions.unsqueeze(0))
    return m, cos, sin


@pytest.mark.parametrize("hd", [64, 128])
def test_rope_matches_hf_qwen2_rotary(hd):
    """Pairing (d, d + hd/2), sign and frequency schedule equal HF's Qwen2 rotary
    embedding (the reference's own end-to-end oracle)."""
    pos = torch.tensor([0, 1, 7, 511, 1023])
    x = torch.randn(5, 3, hd)
    m, cos, sin = _hf_rotary(hd, 1.0e6, pos)
    ref, _ = m.apply_rotary_pos_emb(x.transpose(0, 1).unsqueeze(0), x.transpose(0, 1).unsqueeze(0), cos, sin)
    ref = ref[0].transpose(0, 1)
    got = O.rope_llama(x, pos, 1.0e6)
    torch.testing.assert_close(got, ref, rtol=1e-4, atol=1e-4)


def test_rope_relative_position_property():
    """<R(q, m), R(k, n)> depends only on m - n: catches a wrong sign or pairing even
    without an external library."""
    hd = 128
    q = torch.randn(1, 1, hd, dtype=torch.float64).float()
    k = torch.randn(1, 1, hd, dtype=torch.float64).float()
    dots = []
    for shift in [0, 3, 50, 300]:
        rq = O.rope_llama(q, torch.tensor([100 + shift]), 1.0e4)
        rk = O.rope_llama(k, torch.tensor([40 + shift]), 1.0e4)
        dots.append(float((rq * rk).sum()))
    assert max(dots) - min(dots) < 1e-3 * (abs(dots[0]) + 1)
    # and position 0 is the identity, norms are preserved
    assert torch.allclose(O.rope_llama(q, torch.tensor([0]), 1e6), q)
    r = O.rope_llama(q, torch.tensor([12345]), 1e6)
    assert abs(float(r.norm()) - float(q.norm())) < 1e-4


def test_mrope_matches_hf_qwen2_5_vl():
    from transformers.models.qwen2_5_vl import modeling_qwen2_5_vl as v

    hd, S, sections = 128, 6, (16, 24, 24)
    x = torch.randn(S, 2, hd).to(torch.bfloat16)
    pos = torch.tensor([[0, 0, 0, 0, 5, 6], [0, 0, 1, 1, 5, 6], [0, 1, 0, 1, 5, 6]], dtype=torch.int32)
    inv = O.rope_inv_freq(hd, 1.0e6).double()
    freqs = pos.double().unsqueeze(-1) * inv          # [3, S, hd/2]
    emb = torch.cat([freqs, freqs], -1)                # [3, S, hd]
    cos, sin = emb.cos().unsqueeze(1), emb.sin().unsqueeze(1)  # [3, 1(batch), S, hd]
    xq = x.double().transpose(0, 1).unsqueeze(0)       # [1, H, S, hd]
    ref, _ = v.apply_multimodal_rotary_pos_emb(xq, xq, cos, sin, list(sections))
    ref = ref[0].transpose(0, 1)
    got = O.mrope(x, pos, sections, 1.0e6)
    torch.testing.assert_close(got.float(), ref.float(), rtol=1e-2, atol=1e-2)
    # equal position rows reduce M-RoPE to RoPE-Llama
    p1 = torch.tensor([3, 9, 27])
    same = O.mrope(x[:3], p1.unsqueeze(0).expand(3, 3), sections, 1.0e6)
    torch.testing.assert_close(same, O.rope_llama(x[:3], p1, 1.0e6).to(torch.bfloat16), rtol=0, atol=0)


# ----------------------------------------------------------------------------------
def _brute_attention(q, k, v, qpos, kpos, theta, causal_limit):
    """Pure-Python float64 attention with explicit rotation loops (tiny sizes)."""
    S, Hq, hd = q.shape
    L, Hkv, _ = k.shape
    G = Hq // Hkv
    h2 = hd // 2

    def rot(vec, p):
        out = [0.0] * hd
        for d in range(h2):
            ang = float(np.float32(np.float32(p) * np.float32(1.0 / theta ** (2 * d / hd))))
            c, s = math.cos(ang), math.sin(ang)
            out[d] = vec[d] * c - vec[d + h2] * s
            out[d + h2] = vec[d + h2] * c + vec[d] * s
        return out

    out = np.zeros((S, Hq, hd))
    for i in range(S):
        for h in range(Hq):
            g = h // G
            qi = rot([float(t) for t in q[i, h]], qpos[i])
            sc = []
            for j in range(L):
                if causal_limit is not None and j > i + causal_limit:
                    continue
                kj = rot([float(t) for t in k[j, g]], kpos[j])
                sc.append((j, sum(a * b for a, b in zip(qi, kj)) / math.sqrt(hd)))
            mx = max(s for _, s in sc)
            den = sum(math.exp(s - mx) for _, s in sc)
            for j, s in sc:
                out[i, h] += math.exp(s - mx) / den * v[j, g].double().numpy()
    return out


def test_attention_decode_brute_force():
    q = torch.randn(1, 4, 8).to(torch.bfloat16)
    k = torch.randn(6, 2, 8).to(torch.bfloat16)
    v = torch.randn(6, 2, 8).to(torch.bfloat16)
    ctx = O.AttnCtx(4, 2, 8, rope_theta=1.0e4)
    got = O.attention_decode(q, k, v, 5, ctx)
    ref = _brute_attention(q, k[:5], v[:5], [4], list(range(5)), 1.0e4, None)
    assert np.allclose(_np(got), ref, rtol=1e-2, atol=1e-2)


def test_attention_prefill_brute_force_with_prefix():
    S, L = 3, 7  # 4 prefix rows already in the cache
    q = torch.randn(S, 4, 8).to(torch.bfloat16)
    k = torch.randn(L, 2, 8).to(torch.bfloat16)
    v = torch.randn(L, 2, 8).to(torch.bfloat16)
    ctx = O.AttnCtx(4, 2, 8, rope_theta=1.0e4, q_rope_pos_offset=L - S)
    got = O.attention_prefill(q, k, v, ctx, causal=True)
    ref = _brute_attention(q, k, v, [L - S + i for i in range(S)], list(range(L)), 1.0e4, L - S)
    assert np.allclose(_np(got), ref, rtol=1e-2, atol=1e-2)


def test_attention_matches_torch_sdpa_on_prerotated_inputs():
    S, Hq, Hkv, hd = 9, 6, 2, 64
    q = torch.randn(S, Hq, hd).to(torch.bfloat16)
    k = torch.randn(S, Hkv, hd).to(torch.bfloat16)
    v = torch.randn(S, Hkv, hd).to(torch.bfloat16)
    ctx = O.AttnCtx(Hq, Hkv, hd)
    got = O.attention_prefill(q, k, v, ctx, causal=True)
    qr = O.rope_llama(q, torch.arange(S), 1e6)
    kr = O.rope_llama(k, torch.arange(S), 1e6).repeat_interleave(3, 1)
    vr = v.float().repeat_interleave(3, 1)
    ref = torch.nn.functional.scaled_dot_product_attention(qr.transpose(0, 1), kr.transpose(0, 1),
                                                           vr.transpose(0, 1), is_causal=True).transpose(0, 1)
    torch.testing.assert_close(got.float(), ref, rtol=1e-2, atol=1e-2)


def test_split_kv_merge_equals_unsplit():
    s = np.random.RandomState(0).randn(37)
    vals = np.random.RandomState(1).randn(37, 4)
    full = (np.exp(s - s.max())[:, None] * vals).sum(0) / np.exp(s - s.max()).sum()
    parts = []
    for lo, hi in [(0, 10), (10, 11), (11, 37)]:
        m = s[lo:hi].max()
        p = np.exp(s[lo:hi] - m)
        parts.append(((p[:, None] * vals[lo:hi]).sum(0), m, p.sum()))
    assert np.allclose(O.split_kv_merge(parts), full, rtol=1e-12)


# ----------------------------------------------------------------------------------
def test_embedding_brute_force():
    table = torch.randn(10, 8).to(torch.bfloat16)
    custom = torch.randn(3, 8).to(torch.bfloat16)
    ids = torch.tensor([0, 9, 10, -3, 5, 6, 7, 8], dtype=torch.int32)
    out = O.embedding(ids, table, custom, embed_token_id=6)
    assert torch.equal(out[0], table[0]) and torch.equal(out[1], table[9])
    assert out[2].abs().sum() == 0 and out[3].abs().sum() == 0
    assert torch.equal(out[4], table[5])
    assert torch.equal(out[5], custom[0]) and torch.equal(out[6], custom[1]) and torch.equal(out[7], custom[2])


def test_argmax_ties_lowest_index():
    x = torch.tensor([[1.0, 3.0, 3.0, 2.0], [5.0, 5.0, 5.0, 5.0], [-1.0, -2.0, -1.0, -5.0]])
    assert O.argmax_lowest(x).tolist() == [1, 0, 0]


# ----------------------------------------------------------------------------------
TINY = O.QwenConfig(hidden=64, layers=2, heads=4, kv_heads=2, head_dim=16, inter=96, vocab=211)


def _hf_model(cfg, weights):
    from transformers import Qwen2Config, Qwen2ForCausalLM

    hc = Qwen2Config(hidden_size=cfg.hidden, intermediate_size=cfg.inter, num_hidden_layers=cfg.layers,
                     num_attention_heads=cfg.heads, num_key_value_heads=cfg.kv_heads, head_dim=cfg.head_dim,
                     vocab_size=cfg.vocab, rms_norm_eps=cfg.eps, tie_word_embeddings=cfg.tied,
                     rope_parameters={"rope_type": "default", "rope_theta": cfg.theta}, max_position_embeddings=4096,
                     attn_implementation="eager")
    model = Qwen2ForCausalLM(hc).eval()
    sd = {k: v.float() for k, v in weights.items()}
    missing, unexpected = model.load_state_dict(sd, strict=False)
    assert not unexpected and all(k == "lm_head.weight" for k in missing), (missing, unexpected)
    return model


def test_qwen2_forward_matches_hf_transformers():
    """Op order, residual flow, fused layouts, q/k/v bias, tied LM head and RoPE all
    agree with HF Qwen2ForCausalLM (fp32) on a tiny random model."""
    w = O.random_weights(TINY, seed=3, std=0.2)
    orc = O.Qwen2Oracle(TINY, O.fuse_weights(TINY, w), max_tokens=64)
    ids = torch.randint(0, TINY.vocab, (12,), generator=torch.Generator().manual_seed(1)).to(torch.int32)
    st = orc.new_state()
    got = orc.forward(st, ids)
    model = _hf_model(TINY, w)
    with torch.no_grad():
        ref = model(ids.long().unsqueeze(0)).logits[0, -1]
    rel = float((got - ref).norm() / ref.norm())
    assert rel < 3e-2, rel
    # decode step after prefill == one longer prefill (KV cache write + RoPE position)
    nxt = torch.tensor([7], dtype=torch.int32)
    got2 = orc.forward(st, nxt)
    with torch.no_grad():
        ref2 = model(torch.cat([ids, nxt]).long().unsqueeze(0)).logits[0, -1]
    assert float((got2 - ref2).norm() / ref2.norm()) < 3e-2


def test_qwen2_greedy_matches_hf_generate():
    w = O.random_weights(TINY, seed=5, std=0.2)
    orc = O.Qwen2Oracle(TINY, O.fuse_weights(TINY, w), max_tokens=64)
    prompt = torch.randint(0, TINY.vocab, (8,), generator=torch.Generator().manual_seed(2)).to(torch.int32)
    steps = orc.generate_greedy(prompt, 10)
    model = _hf_model(TINY, w)
    ids = prompt.long().unsqueeze(0)
    for tok, margin in steps:
        with torch.no_grad():
            logits = model(ids).logits[0, -1]
        hf_tok = int(torch.argmax(logits))
        if margin > 0.05:
            assert tok == hf_tok
        ids = torch.cat([ids, torch.tensor([[tok]])], 1)


def test_generate_token_cap():
    """max_generated = min(max_new_tokens, max_tokens - len(prompt) + 1)
    (scheduler.cpp:123-134)."""
    w = O.random_weights(TINY, seed=1)
    orc = O.Qwen2Oracle(TINY, O.fuse_weights(TINY, w), max_tokens=12)
    steps = orc.generate_greedy(torch.arange(8, dtype=torch.int32), 100)
    assert len(steps) == 12 - 8 + 1


# ----------------------------------------------------------------------------------
# SageAttention-style int8 path (no reference implementation: pinned by exact integer
# brute force, quantisation error bounds, the softmax shift invariance K smoothing
# relies on, and agreement with the bf16 attention).
def test_sage_int32_scores_brute_force():
    g = torch.Generator().manual_seed(0)
    q8 = torch.randint(-127, 128, (3, 4, 8), generator=g).to(torch.int8)
    k8 = torch.randint(-127, 128, (5, 2, 8), generator=g).to(torch.int8)
    s = O.sage_scores_int32(q8, k8, 2)
    for h in range(4):
        for i in range(3):
            for j in range(5):
                ref = sum(int(q8[i, h, d]) * int(k8[j, h // 2, d]) for d in range(8))
                assert int(s[h, i, j]) == ref


def test_sage_quant_blocks_bounds_and_rounding():
    x = torch.randn(300, 3, 16) * 3
    x[128:256, 1] = 0.0  # an all-zero (block, head)
    q8, sc = O.sage_quant_blocks(x)
    assert sc.shape == (3, 3) and float(sc[1, 1]) == 1.0 and q8[128:256, 1].abs().sum() == 0
    for b in range(3):
        xb = x[b * 128:(b + 1) * 128]
        amax = xb.abs().amax(dim=(0, 2))
        for h in range(3):
            if float(amax[h]) > 0:
                assert float(sc[b, h]) == float(np.float32(amax[h]) / np.float32(127.0))
        deq = q8[b * 128:(b + 1) * 128].float() * sc[b][None, :, None]
        assert float((deq - xb).abs().max()) <= float(sc[b].max()) * 0.5 + 1e-6
    assert int(q8.abs().max()) <= 127
    # round half to even at exact ties
    t = torch.tensor([[[127.0, 0.5, 1.5, -2.5, 2.5]]])
    q, s = O.sage_quant_blocks(t)
    assert float(s[0, 0]) == 1.0 and q.flatten().tolist() == [127, 0, 2, -2, 2]


def test_sage_kmean_closed_form():
    """sage_kmean is the per-(KV head, channel) mean over tokens: a float64 numpy mean
    over axis 0 rounded once to fp32, exactly; a hand-worked case; the smoothed keys have a
    zero token mean. A sum without the division, a mean over the wrong axis or an fp32
    accumulation fails one of these."""
    torch.manual_seed(4)
    k = (torch.randn(333, 4, 128) * 3 + 1.5).to(torch.bfloat16)
    m = O.sage_kmean(k)
    ref = np.mean(k.float().numpy().astype(np.float64), axis=0).astype(np.float32)
    assert m.shape == (4, 128) and m.dtype == torch.float32
    assert np.array_equal(m.numpy(), ref)
    # tokens 1, 2, 4 of one channel: 7/3 rounded to fp32; a constant channel keeps its value
    t = torch.zeros(3, 1, 2, dtype=torch.bfloat16)
    t[:, 0, 0] = torch.tensor([1.0, 2.0, 4.0])
    t[:, 0, 1] = -0.75
    mt = O.sage_kmean(t)
    assert float(mt[0, 0]) == float(np.float32(7.0 / 3.0)) and float(mt[0, 1]) == -0.75
    # fp32 accumulation of 2^24 + 1 + 1 + ... would lose the ones; float64 keeps them
    big = torch.ones(4097, 1, 1, dtype=torch.bfloat16)
    big[0] = 2.0 ** 24
    assert float(O.sage_kmean(big)[0, 0]) == float(np.float32((2.0 ** 24 + 4096) / 4097))
    ks = k.float() - m[None]
    assert float(ks.double().mean(0).abs().max()) < 1e-5


def test_sage_k_smoothing_is_softmax_invariant():
    """Adding a per-channel constant to K does not change the (exact) attention, which is
    what makes subtracting the K mean legal; the oracle's result barely moves."""
    torch.manual_seed(1)
    q = torch.randn(64, 4, 64).to(torch.bfloat16)
    k = torch.randn(64, 2, 64).to(torch.bfloat16)
    v = torch.randn(64, 2, 64).to(torch.bfloat16)
    shift = (torch.randn(1, 2, 64) * 4).to(torch.bfloat16).float()
    k2 = (k.float() + shift).to(torch.bfloat16)
    o1 = O.sage_attention(q, k, v, 2).float()
    o2 = O.sage_attention(q, k2, v, 2).float()
    assert float((o1 - o2).abs().mean()) < 5e-3


def test_sage_attention_close_to_bf16_attention():
    torch.manual_seed(2)
    q = torch.randn(200, 4, 128).to(torch.bfloat16)
    k = torch.randn(260, 2, 128).to(torch.bfloat16)
    v = torch.randn(260, 2, 128).to(torch.bfloat16)
    o = O.sage_attention(q, k, v, 2).float()
    r = O.attention_prefill(q, k, v, O.AttnCtx(4, 2, 128, rope=False)).float()
    assert float((o - r).abs().mean()) < 5e-3 and float((o - r).abs().max()) < 0.1


# ----------------------------------------------------------------------------------
# Temperature / top-p sampler. The reference's RNG (cuRAND inside un-vendored
# FlashInfer) is not reproducible here, so the oracle is pinned by the published
# Philox4x32-10 known-answer vectors, brute force of the nucleus on tiny rows, and the
# sampled distribution itself (chi-square against softmax(l / T) over the nucleus).
@pytest.mark.parametrize("ctr,key,expect", [
    ((0, 0, 0, 0), (0, 0), (0x6627e8d5, 0xe169c58d, 0xbc57ac4c, 0x9b00dbd8)),
    ((0xffffffff,) * 4, (0xffffffff,) * 2, (0x408f276d, 0x41c83b0e, 0xa20bc7c6, 0x6d5451fd)),
    ((0x243f6a88, 0x85a308d3, 0x13198a2e, 0x03707344), (0xa4093822, 0x299f31d0),
     (0xd16cfe09, 0x94fdcceb, 0x5001e420, 0x24126ea1)),
])
def test_philox4x32_10_known_answers(ctr, key, expect):
    # Random123 kat_vectors, philox4x32_10 (Salmon et al., SC'11)
    assert tuple(O.philox4x32_10(ctr, key)) == expect


def _brute_nucleus(l, T, p):
    """float64 probabilities, sorted descending, smallest prefix with mass >= p (all ties
    of the last value included)."""
    pr = np.exp((l.astype(np.float64) - l.max()) / T)
    pr /= pr.sum()
    order = sorted(range(len(l)), key=lambda i: -pr[i])
    acc, kept = 0.0, []
    for i in order:
        if acc >= p * (1 - 1e-12):
            if pr[i] < pr[kept[-1]]:
                break
        kept.append(i)
        acc += pr[i]
    return set(kept), pr


@pytest.mark.parametrize("seed", range(6))
def test_sampler_nucleus_brute_force(seed):
    rng = np.random.default_rng(seed)
    for T, p in [(0.7, 0.9), (1.0, 0.5), (1.3, 0.95), (0.5, 0.3)]:
        l = (rng.standard_normal(12) * 2).astype(np.float32)
        want, _ = _brute_nucleus(l, T, p)
        e, w = O.sample_masses(l, T)
        tau = O.nucleus_threshold(e, w, p)
        got = set(np.nonzero(e >= tau)[0].tolist())
        assert got == want, (T, p, sorted(got), sorted(want))
    # ties on the boundary value are all kept
    l = np.array([3.0, 1.0, 1.0, 1.0, -2.0], dtype=np.float32)
    e, w = O.sample_masses(l, 1.0)
    assert set(np.nonzero(e >= O.nucleus_threshold(e, w, 0.8))[0].tolist()) == {0, 1, 2, 3}


@pytest.mark.parametrize("T,p", [(0.7, 1.0), (0.7, 0.9), (1.5, 0.6)])
def test_sampler_distribution_chi_square(T, p):
    from scipy.stats import chisquare
    l = np.array([2.0, 1.5, 1.0, 0.4, 0.0, -0.5, -1.0, -3.0], dtype=np.float32)
    keep, pr = _brute_nucleus(l, T, p) if p < 1 else (set(range(len(l))), None)
    if pr is None:
        pr = np.exp((l.astype(np.float64) - l.max()) / T)
        pr /= pr.sum()
    n = 20000
    counts = np.zeros(len(l))
    for off in range(n):
        tok, _ = O.sample_top_p(l, T, p, seed=1234, offset=off)
        counts[tok] += 1
    ids = sorted(keep)
    assert counts[[i for i in range(len(l)) if i not in keep]].sum() == 0
    expect = pr[ids] / pr[ids].sum() * n
    assert chisquare(counts[ids], expect).pvalue > 1e-4


def test_sampler_offsets_and_seeds_draw_fresh_numbers():
    bits = [O.sampling_bits(7, off) for off in range(4096)]
    assert len(set(bits)) > 4000
    assert abs(np.mean(bits) / 2 ** 24 - 0.5) < 0.02
    assert O.sampling_bits(7, 3) != O.sampling_bits(8, 3)
    assert O.sampling_bits(1 << 40, 3) != O.sampling_bits(0, 3)   # high seed word is used
    assert O.sampling_bits(7, 1 << 33) != O.sampling_bits(7, 0)   # high offset word is used
