"""Layer tier through the `edge_fm` bindings, built the way the reference's layer tests
build them (tests/layers/test_*.py: an engine config naming a model directory, a layer
constructed from the config path, torch tensors handed over with
`edge_fm.Tensor.from_dlpack(t.__dlpack__())` and read back with
`torch.from_dlpack(out.to_dlpack())`). The reference checks against FlashInfer; these
check against the oracle (bf16 storage, fp32 math, the same rounding points) at
rtol = atol = 2e-2 for bf16 outputs, exactly for integer outputs (tokens, ids, pointers).

The checkpoint is a small seeded random Qwen2.5-shaped model written as
model.safetensors, so the layers load their weights from a file as the reference's do.
bf16 only: the MI355X kernels compute in bf16 (the reference tests also run fp16)."""
import json
import os

import pytest
import torch

import edge_fm
import efm_setup as S
from oracle import efm_oracle as O
from _util import assert_close_bf16

TOL = dict(rtol=2e-2, atol=2e-2)
CFG = O.QwenConfig(hidden=512, layers=2, heads=4, kv_heads=2, head_dim=128, inter=1024, vocab=3000, tied=False)


def to_efm(t):
    return edge_fm.Tensor.from_dlpack(t.contiguous().__dlpack__())


def from_efm(e):
    return torch.from_dlpack(e.to_dlpack())


@pytest.fixture(scope="module")
def model(tmp_path_factory):
    d = str(tmp_path_factory.mktemp("layer_model"))
    S.write_model_dir(d, S.ModelShape(CFG.hidden, CFG.layers, CFG.heads, CFG.kv_heads, CFG.head_dim, CFG.inter,
                                      CFG.vocab, tied=False))
    w = O.random_weights(CFG, seed=11)
    S.write_checkpoint(d, w)
    cfg_path = os.path.join(d, "engine_config.json")
    S.write_engine_config(cfg_path, d, max_tokens=256, prefix_token_ids=[5, 6, 7])
    return d, cfg_path, w


@pytest.fixture
def fresh_loader():
    """Each layer loads the checkpoint itself, as after the reference tests' clear_stage."""
    loader = edge_fm.WeightLoader.instance()
    loader.clear_stage(edge_fm.ModelStage.Prefill)
    loader.clear_stage(edge_fm.ModelStage.Decode)
    yield loader
    loader.clear_stage(edge_fm.ModelStage.Prefill)


def sampler_config(tmp_path, vocab, temperature, seed=42, top_p=1.0):
    d = tmp_path / f"sampler_{vocab}"
    d.mkdir(exist_ok=True)
    (d / "config.json").write_text(json.dumps({"vocab_size": vocab}))
    p = d / "engine_config.json"
    p.write_text(json.dumps({"model_name": "Qwen2.5", "runtime": {"device": "gpu", "device_id": 0},
                             "prefill_model_path": str(d),
                             "sampling": {"temperature": temperature, "seed": seed, "top_p": top_p}}))
    return str(p)


def attention_config(tmp_path, hq, hkv, hd):
    """tests/layers/test_attn.py:23-55: a config.json with the head counts only."""
    d = tmp_path / f"attn_{hq}_{hkv}_{hd}"
    d.mkdir(exist_ok=True)
    (d / "config.json").write_text(json.dumps({"num_attention_heads": hq, "num_key_value_heads": hkv,
                                               "hidden_size": hq * hd, "rope_theta": 1000000.0,
                                               "torch_dtype": "bfloat16"}))
    p = d / "engine_config.json"
    p.write_text(json.dumps({"model_name": "Qwen2.5", "runtime": {"device": "gpu", "device_id": 0},
                             "prefill_model_path": str(d)}))
    return str(p)


# ---------------------------------------------------------------------------------
# Tensor DLPack import (pybind_debug.cpp:437-449: the data is copied)
# ---------------------------------------------------------------------------------
@pytest.mark.gpu
def test_tensor_from_dlpack_copies(gpu):
    t = torch.randn(3, 5, device=gpu).to(torch.bfloat16)
    e = to_efm(t)
    assert e.shape() == [3, 5] and e.dtype() == edge_fm.DType.BFloat16
    assert e.data_ptr() != t.data_ptr()
    back = from_efm(e).clone()
    t.zero_()
    torch.cuda.synchronize()
    assert torch.equal(from_efm(e), back) and back.abs().sum() > 0
    ids = torch.arange(7, dtype=torch.int32, device=gpu)
    assert torch.equal(from_efm(to_efm(ids)), ids)
    with pytest.raises(Exception):
        edge_fm.Tensor.from_dlpack(t.t().__dlpack__())   # not row-major


# ---------------------------------------------------------------------------------
# RMSNormLayer (tests/layers/test_layernorm.py)
# ---------------------------------------------------------------------------------
@pytest.mark.gpu
@pytest.mark.parametrize("batch_size", [1, 32, 64, 128])
def test_rmsnorm_layer(gpu, model, fresh_loader, batch_size):
    _, cfg_path, w = model
    layer = edge_fm.RMSNormLayer(layer_id=0, config_path=cfg_path)
    assert layer.layer_role() == "input_norm"
    torch.manual_seed(42)
    x = torch.randn(batch_size, CFG.hidden, dtype=torch.bfloat16)
    out = to_efm(torch.empty(batch_size, CFG.hidden, dtype=torch.bfloat16, device=gpu))
    layer.forward_rmsnorm(to_efm(x.to(gpu)), out)
    torch.cuda.synchronize()
    assert_close_bf16(from_efm(out), O.rms_norm(x, w["model.layers.0.input_layernorm.weight"], CFG.eps), **TOL,
                      what="forward_rmsnorm")


@pytest.mark.gpu
@pytest.mark.parametrize("weight_type,name", [("input", "model.layers.1.input_layernorm.weight"),
                                              ("post_attention", "model.layers.1.post_attention_layernorm.weight"),
                                              ("final", "model.norm.weight")])
def test_fused_add_rmsnorm_layer(gpu, model, fresh_loader, weight_type, name):
    _, cfg_path, w = model
    layer = edge_fm.RMSNormLayer(layer_id=1, config_path=cfg_path, weight_type=weight_type)
    torch.manual_seed(7)
    x = torch.randn(33, CFG.hidden, dtype=torch.bfloat16)
    r = torch.randn(33, CFG.hidden, dtype=torch.bfloat16)
    inout, res = to_efm(x.to(gpu)), to_efm(r.to(gpu))
    layer.forward_fused_add_rmsnorm(inout, res)
    torch.cuda.synchronize()
    exp_out, exp_res = O.fused_add_rms_norm(x, r, w[name], CFG.eps)
    assert_close_bf16(from_efm(inout), exp_out, **TOL, what="fused_add_rmsnorm inout")
    assert torch.equal(from_efm(res).cpu(), exp_res), "residual = bf16(x + residual) exactly"


@pytest.mark.gpu
def test_rmsnorm_layer_rejects_bad_shapes(gpu, model, fresh_loader):
    _, cfg_path, _ = model
    layer = edge_fm.RMSNormLayer(0, cfg_path)
    bad = to_efm(torch.zeros(4, CFG.hidden + 8, dtype=torch.bfloat16, device=gpu))
    with pytest.raises(edge_fm.InvalidRequestError):
        layer.forward_rmsnorm(bad, bad)
    with pytest.raises(edge_fm.ConfigurationError):
        edge_fm.RMSNormLayer(7, cfg_path)   # no such layer in the checkpoint


# ---------------------------------------------------------------------------------
# ActivationLayer (tests/layers/test_activation.py)
# ---------------------------------------------------------------------------------
@pytest.mark.gpu
@pytest.mark.parametrize("shape", [(1,), (7,), (64,), (2, 5)])
def test_activation_layer(gpu, model, shape):
    _, cfg_path, _ = model
    layer = edge_fm.ActivationLayer(cfg_path)
    torch.manual_seed(3)
    x = torch.randn(*shape, 2 * CFG.inter, dtype=torch.bfloat16)
    for fn, up_first in (("forward_silu_and_mul", False), ("forward_silu_and_mul_up_gate", True)):
        out = to_efm(torch.empty(*shape, CFG.inter, dtype=torch.bfloat16, device=gpu))
        getattr(layer, fn)(to_efm(x.to(gpu)), out)
        torch.cuda.synchronize()
        assert_close_bf16(from_efm(out), O.act_and_mul(x, up_first=up_first), **TOL, what=fn)
    with pytest.raises(edge_fm.InvalidRequestError):
        layer.forward_silu_and_mul(to_efm(x.to(gpu)), to_efm(torch.empty(*shape, 8, dtype=torch.bfloat16,
                                                                          device=gpu)))


# ---------------------------------------------------------------------------------
# AttentionLayer (tests/layers/test_attn.py: RoPE-Llama on read, theta 1e6)
# ---------------------------------------------------------------------------------
PREFILL_CASES = [(128, 512, 16, 16, 128, True), (256, 1024, 16, 8, 128, True), (64, 256, 16, 16, 64, False),
                 (200, 200, 12, 2, 128, True)]
DECODE_CASES = [(512, 4, 4, 128), (1024, 8, 8, 128), (2048, 16, 8, 128), (700, 14, 2, 64)]


@pytest.mark.gpu
@pytest.mark.parametrize("qo,kv,hq,hkv,hd,causal", PREFILL_CASES)
def test_attention_layer_prefill(gpu, tmp_path, qo, kv, hq, hkv, hd, causal):
    layer = edge_fm.AttentionLayer(attention_config(tmp_path, hq, hkv, hd))
    torch.manual_seed(42)
    q = torch.randn(qo, hq, hd, dtype=torch.bfloat16)
    k = torch.randn(kv, hkv, hd, dtype=torch.bfloat16)
    v = torch.randn(kv, hkv, hd, dtype=torch.bfloat16)
    o = to_efm(torch.empty(qo, hq, hd, dtype=torch.bfloat16, device=gpu))
    layer.forward_prefill(to_efm(q.to(gpu)), to_efm(k.to(gpu)), to_efm(v.to(gpu)), o, causal=causal)
    torch.cuda.synchronize()
    exp = O.attention_prefill(q, k, v, O.AttnCtx(hq, hkv, hd), causal=causal)
    assert_close_bf16(from_efm(o), exp, **TOL, what="AttentionLayer.forward_prefill")


@pytest.mark.gpu
@pytest.mark.parametrize("kv,hq,hkv,hd", DECODE_CASES)
def test_attention_layer_decode(gpu, tmp_path, kv, hq, hkv, hd):
    layer = edge_fm.AttentionLayer(attention_config(tmp_path, hq, hkv, hd))
    torch.manual_seed(42)
    q = torch.randn(1, hq, hd, dtype=torch.bfloat16)
    k = torch.randn(kv, hkv, hd, dtype=torch.bfloat16)
    v = torch.randn(kv, hkv, hd, dtype=torch.bfloat16)
    o = to_efm(torch.empty(1, hq, hd, dtype=torch.bfloat16, device=gpu))
    kd, vd = to_efm(k.to(gpu)), to_efm(v.to(gpu))
    layer.forward_decode(to_efm(q.to(gpu)), kd, vd, o)
    torch.cuda.synchronize()
    exp = O.attention_decode(q, k, v, kv, O.AttnCtx(hq, hkv, hd))
    assert_close_bf16(from_efm(o), exp, **TOL, what="AttentionLayer.forward_decode")
    # device-side length over a longer cache (graph-stable decode form)
    live = kv // 2 + 3
    d_len = to_efm(torch.tensor([live], dtype=torch.int32, device=gpu))
    o2 = to_efm(torch.empty(1, hq, hd, dtype=torch.bfloat16, device=gpu))
    layer.forward_decode(to_efm(q.to(gpu)), kd, vd, o2, 0, kv, d_len)
    torch.cuda.synchronize()
    exp2 = O.attention_decode(q, k, v, live, O.AttnCtx(hq, hkv, hd))
    assert_close_bf16(from_efm(o2), exp2, **TOL, what="AttentionLayer.forward_decode(d_kv_len)")


@pytest.mark.gpu
def test_attention_layer_rejects_mismatched_shapes(gpu, tmp_path):
    layer = edge_fm.AttentionLayer(attention_config(tmp_path, 8, 2, 128))
    q = to_efm(torch.zeros(2, 8, 128, dtype=torch.bfloat16, device=gpu))
    kv = to_efm(torch.zeros(16, 4, 128, dtype=torch.bfloat16, device=gpu))
    with pytest.raises(edge_fm.InvalidRequestError):
        layer.forward_prefill(q, kv, kv, q)
    with pytest.raises(edge_fm.InvalidRequestError):
        layer.forward_decode(q, kv, kv, q)   # decode q must be [1, Hq, hd]


# ---------------------------------------------------------------------------------
# SamplerLayer (tests/layers/test_sampler.py)
# ---------------------------------------------------------------------------------
@pytest.mark.gpu
@pytest.mark.parametrize("batch_size", [1, 4, 32])
@pytest.mark.parametrize("vocab", [1000, 151936])
def test_sampler_layer_greedy(gpu, tmp_path, batch_size, vocab):
    layer = edge_fm.SamplerLayer(sampler_config(tmp_path, vocab, 0.0, seed=0))
    torch.manual_seed(batch_size + vocab)
    logits = torch.randn(batch_size, vocab)
    ids = to_efm(torch.zeros(batch_size, dtype=torch.int32, device=gpu))
    layer.forward(to_efm(logits.to(gpu)), ids)
    torch.cuda.synchronize()
    assert torch.equal(from_efm(ids).cpu(), O.argmax_lowest(logits))


@pytest.mark.gpu
def test_sampler_layer_greedy_edge_cases(gpu, tmp_path):
    """tests/layers/test_sampler.py:148-205: ties go to the lowest id, a single large
    logit wins anywhere in the row, a row of -1e9 gives 0."""
    vocab = 32000
    layer = edge_fm.SamplerLayer(sampler_config(tmp_path, vocab, 0.0, seed=0))
    rows = [torch.zeros(vocab), torch.ones(vocab), torch.full((vocab,), -1e9)]
    for pos in (0, vocab // 2, vocab - 1):
        r = torch.zeros(vocab)
        r[pos] = 1.0
        rows.append(r)
    logits = torch.stack(rows)
    ids = to_efm(torch.zeros(len(rows), dtype=torch.int32, device=gpu))
    layer.forward(to_efm(logits.to(gpu)), ids)
    torch.cuda.synchronize()
    assert from_efm(ids).cpu().tolist() == [0, 0, 0, 0, vocab // 2, vocab - 1]


@pytest.mark.gpu
@pytest.mark.parametrize("temperature", [0.5, 1.0, 1.5])
@pytest.mark.parametrize("top_p", [1.0, 0.9])
def test_sampler_layer_sampling(gpu, tmp_path, temperature, top_p):
    """Row b draws with Philox counter b and the configured seed: every draw equals the
    oracle's, and a second call repeats the first (fixed seed and offset)."""
    vocab, batch, seed = 4096, 6, 42
    layer = edge_fm.SamplerLayer(sampler_config(tmp_path, vocab, temperature, seed=seed, top_p=top_p))
    torch.manual_seed(int(temperature * 10) + int(top_p * 100))
    logits = torch.randn(batch, vocab) * 3
    lg = to_efm(logits.to(gpu))
    ids = to_efm(torch.zeros(batch, dtype=torch.int32, device=gpu))
    layer.forward(lg, ids)
    torch.cuda.synchronize()
    got = from_efm(ids).cpu().tolist()
    exp = [O.sample_top_p(logits[b], temperature, top_p, seed, b)[0] for b in range(batch)]
    assert got == exp
    ids2 = to_efm(torch.zeros(batch, dtype=torch.int32, device=gpu))
    layer.forward(lg, ids2)
    torch.cuda.synchronize()
    assert from_efm(ids2).cpu().tolist() == got


@pytest.mark.gpu
def test_sampler_layer_rejects_bad_inputs(gpu, tmp_path):
    layer = edge_fm.SamplerLayer(sampler_config(tmp_path, 1000, 0.0))
    ids = to_efm(torch.zeros(2, dtype=torch.int32, device=gpu))
    with pytest.raises(edge_fm.InvalidRequestError):
        layer.forward(to_efm(torch.zeros(2, 999, device=gpu)), ids)             # vocab mismatch
    with pytest.raises(edge_fm.InvalidRequestError):
        layer.forward(to_efm(torch.zeros(2, 1000, dtype=torch.bfloat16, device=gpu)), ids)   # not fp32


# ---------------------------------------------------------------------------------
# EmbedHeadLayer (tests/layers/test_embed.py)
# ---------------------------------------------------------------------------------
@pytest.mark.gpu
def test_embed_head_layer(gpu, model, fresh_loader):
    _, cfg_path, w = model
    layer = edge_fm.EmbedHeadLayer(cfg_path)
    table = w["model.embed_tokens.weight"]
    ids = torch.tensor([[0, 5, CFG.vocab - 1, CFG.vocab, 17, -3], [9, 9, 100, 2999, 1, 2]], dtype=torch.int32)
    out = to_efm(torch.empty(2, 6, CFG.hidden, dtype=torch.bfloat16, device=gpu))
    layer.forward_for_tokens(to_efm(ids.to(gpu)), out)
    torch.cuda.synchronize()
    exp = O.embedding(ids.flatten(), table).reshape(2, 6, CFG.hidden)
    assert torch.equal(from_efm(out).cpu(), exp)
    # custom rows for ids [2990, 2993)
    custom = torch.randn(3, CFG.hidden).to(torch.bfloat16)
    ids2 = torch.tensor([[2989, 2990, 2991, 2992, 2993, 4]], dtype=torch.int32)
    out2 = to_efm(torch.empty(1, 6, CFG.hidden, dtype=torch.bfloat16, device=gpu))
    layer.forward_for_embeddings(to_efm(ids2.to(gpu)), to_efm(custom.to(gpu)), out2, embed_token_id=2990)
    torch.cuda.synchronize()
    exp2 = O.embedding(ids2.flatten(), table, custom, 2990).reshape(1, 6, CFG.hidden)
    assert torch.equal(from_efm(out2).cpu(), exp2)
    with pytest.raises(edge_fm.InvalidRequestError):
        layer.forward_for_tokens(to_efm(ids.flatten().to(gpu)), out)   # ids must be [batch, seq]


# ---------------------------------------------------------------------------------
# LinearLayer and the fused projections (tests/layers/test_linear.py)
# ---------------------------------------------------------------------------------
@pytest.mark.gpu
@pytest.mark.parametrize("m,stage", [(1, "Decode"), (1, "Prefill"), (64, "Prefill"), (200, "Prefill")])
def test_linear_layer(gpu, model, fresh_loader, m, stage):
    _, cfg_path, w = model
    prefix = "model.layers.0.mlp.down_proj"
    layer = edge_fm.LinearLayer(prefix, cfg_path, CFG.inter, CFG.hidden)
    torch.manual_seed(m)
    x = torch.randn(m, CFG.inter, dtype=torch.bfloat16)
    out = to_efm(torch.empty(m, CFG.hidden, dtype=torch.bfloat16, device=gpu))
    layer.forward_fp16_bf16(to_efm(x.to(gpu)), out, 0, stage)
    torch.cuda.synchronize()
    assert_close_bf16(from_efm(out), O.linear(x, w[prefix + ".weight"]), **TOL, what=f"LinearLayer m={m}")
    info = json.loads(layer.debug_cached_impl_info(stage, m))
    assert info["selected_impl_id"] and info["layer_role"] == "mlp_down"
    winfo = json.loads(layer.debug_weight_tensor_info(stage))
    assert winfo["weight_shape"] == [CFG.hidden, CFG.inter] and not winfo["has_bias"]


@pytest.mark.gpu
@pytest.mark.parametrize("m", [1, 96])
def test_fused_qkv_linear_layer(gpu, model, fresh_loader, m):
    _, cfg_path, w = model
    base = "model.layers.1.self_attn"
    qd, kvd = CFG.q_dim, CFG.kv_dim
    layer = edge_fm.FusedQKVLinearLayer(base, cfg_path, CFG.hidden, qd, kvd, kvd)
    torch.manual_seed(m + 1)
    x = torch.randn(m, CFG.hidden, dtype=torch.bfloat16)
    out = to_efm(torch.empty(m, qd + 2 * kvd, dtype=torch.bfloat16, device=gpu))
    layer.forward_fp16_bf16(to_efm(x.to(gpu)), out, 0, "Decode" if m == 1 else "Prefill")
    torch.cuda.synchronize()
    wq = torch.cat([w[f"{base}.{p}_proj.weight"] for p in "qkv"])
    bq = torch.cat([w[f"{base}.{p}_proj.bias"] for p in "qkv"])
    assert_close_bf16(from_efm(out), O.linear(x, wq, bq), **TOL, what="FusedQKVLinearLayer")
    assert json.loads(layer.debug_cached_impl_info())["layer_role"] == "fused_qkv"


@pytest.mark.gpu
def test_fused_gate_up_linear_layer(gpu, model, fresh_loader):
    _, cfg_path, w = model
    base = "model.layers.0.mlp"
    I, H = CFG.inter, CFG.hidden
    layer = edge_fm.FusedGateUpLinearLayer(base, cfg_path, H, I, I)
    wug = torch.cat([w[base + ".up_proj.weight"], w[base + ".gate_proj.weight"]])
    for m, stage in ((1, "Decode"), (80, "Prefill")):
        torch.manual_seed(m)
        x = torch.randn(m, H, dtype=torch.bfloat16)
        xd = to_efm(x.to(gpu))
        both = to_efm(torch.empty(m, 2 * I, dtype=torch.bfloat16, device=gpu))
        layer.forward_fp16_bf16(xd, both, 0, stage)
        act = to_efm(torch.empty(m, I, dtype=torch.bfloat16, device=gpu))
        fused = (layer.try_forward_decode_swiglu_fused(xd, act) if m == 1
                 else layer.try_forward_prefill_swiglu_fused(xd, act))
        torch.cuda.synchronize()
        assert fused, f"fused SwiGLU not taken at m={m}"
        assert_close_bf16(from_efm(both), O.linear(x, wug), **TOL, what=f"[up | gate] m={m}")
        assert_close_bf16(from_efm(act), O.gate_up_swiglu(x, wug), **TOL, what=f"fused SwiGLU m={m}")
    # shapes the fused entry points do not take: nothing is done, False is returned
    x8 = to_efm(torch.randn(8, H, device=gpu).to(torch.bfloat16))
    out8 = to_efm(torch.full((8, I), 7.0, device=gpu).to(torch.bfloat16))
    assert not layer.try_forward_prefill_swiglu_fused(x8, out8)      # m < 64
    assert not layer.try_forward_decode_swiglu_fused(x8, out8)       # m != 1
    torch.cuda.synchronize()
    assert bool((from_efm(out8) == 7.0).all())


@pytest.mark.gpu
def test_lm_head_linear_layer(gpu, model, fresh_loader):
    _, cfg_path, w = model
    layer = edge_fm.LMHeadLinearLayer(cfg_path, CFG.hidden, CFG.vocab)
    W = w["lm_head.weight"]
    for seed in range(4):
        torch.manual_seed(100 + seed)
        x = torch.randn(1, CFG.hidden, dtype=torch.bfloat16)
        xd = to_efm(x.to(gpu))
        logits = to_efm(torch.empty(1, CFG.vocab, dtype=torch.float32, device=gpu))
        layer.forward_fp16_bf16(xd, logits, 0, "Decode")
        tok = to_efm(torch.full((1,), -1, dtype=torch.int32, device=gpu))
        assert layer.try_forward_top1(xd, tok)
        torch.cuda.synchronize()
        exp = O.linear(x, W, out_f32=True)
        torch.testing.assert_close(from_efm(logits).cpu(), exp, rtol=2e-2, atol=2e-2)
        top2 = exp[0].topk(2)
        t = int(from_efm(tok).item())
        if float(top2.values[0] - top2.values[1]) > 1e-3:
            assert t == int(top2.indices[0])
        else:
            assert t in top2.indices.tolist()
    tok = to_efm(torch.zeros(1, dtype=torch.int32, device=gpu))
    assert not layer.try_forward_top1(xd, tok, 0, "Prefill")


@pytest.mark.gpu
def test_lm_head_layer_uses_tied_embedding(gpu, tmp_path, fresh_loader):
    """A checkpoint without lm_head.weight ties the head to model.embed_tokens.weight."""
    cfg = O.QwenConfig(hidden=256, layers=1, heads=2, kv_heads=1, head_dim=128, inter=512, vocab=900, tied=True)
    d = str(tmp_path / "tied")
    S.write_model_dir(d, S.ModelShape(cfg.hidden, 1, 2, 1, 128, 512, 900, tied=True))
    w = O.random_weights(cfg, seed=5)
    w.pop("lm_head.weight", None)
    S.write_checkpoint(d, w)
    p = os.path.join(d, "engine_config.json")
    S.write_engine_config(p, d)
    layer = edge_fm.LMHeadLinearLayer(p, cfg.hidden, cfg.vocab)
    x = torch.randn(1, cfg.hidden).to(torch.bfloat16)
    out = to_efm(torch.empty(1, cfg.vocab, dtype=torch.float32, device=gpu))
    layer.forward_fp16_bf16(to_efm(x.to(gpu)), out, 0, "Decode")
    torch.cuda.synchronize()
    torch.testing.assert_close(from_efm(out).cpu(), O.linear(x, w["model.embed_tokens.weight"], out_f32=True),
                               rtol=2e-2, atol=2e-2)


# ---------------------------------------------------------------------------------
# KVManager (kv_manager.cpp:45-262)
# ---------------------------------------------------------------------------------
@pytest.mark.gpu
def test_kv_manager_layout_and_status(gpu, model):
    _, cfg_path, _ = model
    kv = edge_fm.KVManager(cfg_path)
    assert kv.is_request_valid(0) and not kv.is_request_valid(1)
    reads, writes = kv.get_read_kvcache(0), kv.get_write_kvcache(0)
    assert len(reads) == len(writes) == CFG.layers
    layer_bytes = 2 * 256 * CFG.kv_dim * 2          # [K | V] x max_tokens rows x bf16
    assert [r - reads[0] for r in reads] == [l * layer_bytes for l in range(CFG.layers)]
    assert [wr - r for wr, r in zip(writes, reads)] == [3 * CFG.kv_dim * 2] * CFG.layers
    st = kv.get_status()
    assert st.device_id == 0 and len(st.slots) == 1
    s = st.slots[0]
    assert (s.request_id, s.prefix_token_ids, s.prefix_size, s.max_tokens) == (0, [5, 6, 7], 3, 256)
    assert s.allocated_size == CFG.layers * layer_bytes
    with pytest.raises(edge_fm.InvalidRequestError):
        kv.get_read_kvcache(9)
