"""GPU parity tests of every C-ABI operator against the CPU oracle on identical seeded
inputs (ctypes through include/edgefm_hip.h). Shapes are the BASELINE head / layer
shapes: Qwen2.5-0.5B (14/2, hd 64), 1.5B (12/2, hd 128), 3B (16/2), 7B (28/4).
Mirrors tests/operators/test_attention_decode.py, test_norm_sampler.py,
test_decode_linear.py and test_fused_gate_up_activation.py of the reference."""
import math

import pytest
import torch

import efm_capi as C
from oracle import efm_oracle as O
from _util import assert_close_bf16, ptr, stream

pytestmark = pytest.mark.gpu

HEAD_CASES = [
    pytest.param(14, 2, 64, id="0p5b"),
    pytest.param(12, 2, 128, id="1p5b"),
    pytest.param(16, 2, 128, id="3b"),
    pytest.param(28, 4, 128, id="7b"),
]


def _decode(ctx, q, k, v, kv_len, d_kv_len=None, max_kv_len=0):
    ws_bytes = C.load().efm_attention_decode_workspace_bytes(ctx, max_kv_len if d_kv_len is not None else kv_len)
    ws = torch.zeros(max(ws_bytes, 256), dtype=torch.uint8, device=q.device)
    o = torch.empty_like(q)
    C.call("efm_attention_decode", ctx, ptr(q), ptr(k), ptr(v), ptr(o), kv_len, ptr(d_kv_len), max_kv_len,
           ptr(ws), ws.numel(), stream())
    torch.cuda.synchronize()
    return o, ws


@pytest.mark.parametrize("hq,hkv,hd", HEAD_CASES)
@pytest.mark.parametrize("kv_len", [1, 7, 33, 512, 1024, 2048])
def test_attention_decode_matches_oracle(gpu, hq, hkv, hd, kv_len):
    torch.manual_seed(0)
    q = torch.randn(1, hq, hd, dtype=torch.bfloat16)
    k = torch.randn(kv_len, hkv, hd, dtype=torch.bfloat16)
    v = torch.randn(kv_len, hkv, hd, dtype=torch.bfloat16)
    ref = O.attention_decode(q, k, v, kv_len, O.AttnCtx(hq, hkv, hd))
    ctx = C.make_attention_ctx(hq, hkv, hd)
    out, _ = _decode(ctx, q.to(gpu), k.to(gpu), v.to(gpu), kv_len)
    assert_close_bf16(out, ref, what=f"decode hq={hq} hkv={hkv} hd={hd} kv={kv_len}")


@pytest.mark.parametrize("hq,hkv,hd", [pytest.param(28, 4, 128, id="7b")])
def test_attention_decode_long_context(gpu, hq, hkv, hd):
    torch.manual_seed(1)
    kv_len = 16385
    q = torch.randn(1, hq, hd, dtype=torch.bfloat16)
    k = torch.randn(kv_len, hkv, hd, dtype=torch.bfloat16)
    v = torch.randn(kv_len, hkv, hd, dtype=torch.bfloat16)
    ref = O.attention_decode(q, k, v, kv_len, O.AttnCtx(hq, hkv, hd))
    out, _ = _decode(C.make_attention_ctx(hq, hkv, hd), q.to(gpu), k.to(gpu), v.to(gpu), kv_len)
    assert_close_bf16(out, ref, what="decode 16k")


@pytest.mark.parametrize("hq,hkv,hd", HEAD_CASES)
@pytest.mark.parametrize("kv_len", [512, 1024, 2048])
def test_attention_decode_graph_like_path_matches_plain(gpu, hq, hkv, hd, kv_len):
    """d_kv_len + max_kv_len over a larger cache == plain call on the first kv_len rows
    (tests/operators/test_attention_decode.py:155-179). Called twice to check that the
    in-workspace merge counters reset themselves."""
    torch.manual_seed(0)
    max_kv = 2048
    q = torch.randn(1, hq, hd, dtype=torch.bfloat16, device=gpu)
    k = torch.randn(max_kv, hkv, hd, dtype=torch.bfloat16, device=gpu)
    v = torch.randn(max_kv, hkv, hd, dtype=torch.bfloat16, device=gpu)
    ctx = C.make_attention_ctx(hq, hkv, hd)
    d_len = torch.tensor([kv_len], dtype=torch.int32, device=gpu)
    ws_bytes = C.load().efm_attention_decode_workspace_bytes(ctx, max_kv)
    ws = torch.zeros(ws_bytes, dtype=torch.uint8, device=gpu)
    outs = []
    for _ in range(2):
        o = torch.empty_like(q)
        C.call("efm_attention_decode", ctx, ptr(q), ptr(k), ptr(v), ptr(o), 0, ptr(d_len), max_kv, ptr(ws),
               ws.numel(), stream())
        torch.cuda.synchronize()
        outs.append(o)
    plain, _ = _decode(ctx, q, k[:kv_len].contiguous(), v[:kv_len].contiguous(), kv_len)
    assert_close_bf16(outs[0], plain)
    assert torch.equal(outs[0], outs[1])


def test_attention_decode_no_rope_and_prerotated(gpu):
    """pos_encoding NONE equals plain softmax attention; k_already_prerotated with
    pre-rotated K equals RoPE-on-read (tests/operators/test_attention_prefill.py:118-164)."""
    torch.manual_seed(3)
    hq, hkv, hd, L = 12, 2, 128, 300
    q = torch.randn(1, hq, hd, dtype=torch.bfloat16)
    k = torch.randn(L, hkv, hd, dtype=torch.bfloat16)
    v = torch.randn(L, hkv, hd, dtype=torch.bfloat16)
    ref = O.attention_decode(q, k, v, L, O.AttnCtx(hq, hkv, hd, rope=False))
    out, _ = _decode(C.make_attention_ctx(hq, hkv, hd, rope=False), q.to(gpu), k.to(gpu), v.to(gpu), L)
    assert_close_bf16(out, ref, what="no-rope")
    k_rot = O.rope_llama(k, torch.arange(L), 1.0e6).to(torch.bfloat16)
    rot_ref = O.attention_decode(q, k, v, L, O.AttnCtx(hq, hkv, hd))
    out2, _ = _decode(C.make_attention_ctx(hq, hkv, hd, k_already_prerotated=True), q.to(gpu), k_rot.to(gpu),
                      v.to(gpu), L)
    assert_close_bf16(out2, rot_ref, what="prerotated")


@pytest.mark.parametrize("hq,hkv,hd", HEAD_CASES)
@pytest.mark.parametrize("kv_len", [1, 129, 767, 1025, 4099])
@pytest.mark.parametrize("merge", [True, False])
def test_attention_decode_prerotated_except_newest(gpu, hq, hkv, hd, kv_len, merge):
    """EFM_K_PREROTATED_EXCEPT_NEWEST: rows [0, L-1) hold rotated keys, row L-1 the
    un-rotated key of this step. The output equals RoPE-on-read over the un-rotated cache
    (and the oracle), row L-1 is stored back rotated (within one bf16 rounding of the
    oracle's rotation) and no other row changes. Rows >= L of the max_kv_len allocation
    hold NaN: the split loads issued before the length is read must not leak them."""
    torch.manual_seed(kv_len)
    max_kv = kv_len + 77
    q = torch.randn(1, hq, hd, dtype=torch.bfloat16)
    k = torch.randn(kv_len, hkv, hd, dtype=torch.bfloat16)
    v = torch.randn(kv_len, hkv, hd, dtype=torch.bfloat16)
    ref = O.attention_decode(q, k, v, kv_len, O.AttnCtx(hq, hkv, hd))
    k_rot = O.rope_llama(k, torch.arange(kv_len), 1.0e6).to(torch.bfloat16)
    kc = torch.full((max_kv, hkv, hd), float("nan"), dtype=torch.bfloat16)
    vc = torch.full((max_kv, hkv, hd), float("nan"), dtype=torch.bfloat16)
    kc[: kv_len - 1] = k_rot[: kv_len - 1]
    kc[kv_len - 1] = k[kv_len - 1]
    vc[:kv_len] = v
    kc, vc, qg = kc.to(gpu), vc.to(gpu), q.to(gpu)
    ctx = C.make_attention_ctx(hq, hkv, hd)
    ctx.k_already_prerotated = C.EFM_K_PREROTATED_EXCEPT_NEWEST
    d_len = torch.tensor([kv_len], dtype=torch.int32, device=gpu)
    ws = torch.zeros(C.load().efm_attention_decode_workspace_bytes(ctx, max_kv), dtype=torch.uint8, device=gpu)
    if merge:
        o = torch.empty_like(qg)
        C.call("efm_attention_decode", ctx, ptr(qg), ptr(kc), ptr(vc), ptr(o), 0, ptr(d_len), max_kv, ptr(ws),
               ws.numel(), stream())
        torch.cuda.synchronize()
        assert_close_bf16(o, ref, what=f"prerotated-except-newest L={kv_len}")
        plain, _ = _decode(C.make_attention_ctx(hq, hkv, hd), qg, k.to(gpu), v.to(gpu), kv_len)
        assert_close_bf16(o, plain, what="vs rope-on-read")
    else:
        C.call("efm_decode_attention_partials", ctx, ptr(qg), ptr(kc), ptr(vc), ptr(d_len), max_kv, ptr(ws),
               ws.numel(), stream())
        torch.cuda.synchronize()
    got = kc.cpu()
    assert torch.equal(got[: kv_len - 1], k_rot[: kv_len - 1]), "rows before the newest must not change"
    assert torch.isnan(got[kv_len:].float()).all(), "rows past L must not be written"
    assert_close_bf16(got[kv_len - 1], k_rot[kv_len - 1], rtol=1e-2, atol=1e-2, what="newest row stored rotated")


@pytest.mark.parametrize("hq,hkv,hd", HEAD_CASES)
@pytest.mark.parametrize("kv_len,max_kv", [(1, 64), (31, 31), (33, 700), (640, 768), (1025, 1100), (3000, 3000),
                                           (5000, 5000)])
@pytest.mark.parametrize("layout", ["rope_on_read", "rotated_except_newest", "no_rope"])
def test_attention_decode_one_wave_splits(gpu, knob, hq, hkv, hd, kv_len, max_kv, layout):
    """The one-wave split kernel of short and mid contexts (32- and 64-key splits, a
    partial last tile, a single split that writes the output itself) against the oracle
    and against the kernels those lengths ran before it (EFM_KNOB_DECODE_TILE), over the
    three cache layouts: un-rotated keys rotated on read (the reference's), rotated keys
    with this step's row still un-rotated (the engine's), and no RoPE (M-RoPE models).
    Rows >= L hold NaN."""
    torch.manual_seed(kv_len * 7 + hd)
    q = torch.randn(1, hq, hd, dtype=torch.bfloat16)
    k = torch.randn(kv_len, hkv, hd, dtype=torch.bfloat16)
    v = torch.randn(kv_len, hkv, hd, dtype=torch.bfloat16)
    rope = layout != "no_rope"
    ref = O.attention_decode(q, k, v, kv_len, O.AttnCtx(hq, hkv, hd, rope=rope))
    kstore = k
    if layout == "rotated_except_newest":
        kstore = O.rope_llama(k, torch.arange(kv_len), 1.0e6).to(torch.bfloat16)
        kstore[kv_len - 1] = k[kv_len - 1]
    ctx = C.make_attention_ctx(hq, hkv, hd, rope=rope)
    if layout == "rotated_except_newest":
        ctx.k_already_prerotated = C.EFM_K_PREROTATED_EXCEPT_NEWEST
    d_len = torch.tensor([kv_len], dtype=torch.int32, device=gpu)
    ws = torch.zeros(C.load().efm_attention_decode_workspace_bytes(ctx, max_kv), dtype=torch.uint8, device=gpu)
    qg = q.to(gpu)
    outs, caches = [], []
    for tile_off in (0, 1):
        knob(C.EFM_KNOB_DECODE_TILE, tile_off)
        kc = torch.full((max_kv, hkv, hd), float("nan"), dtype=torch.bfloat16)
        vc = torch.full((max_kv, hkv, hd), float("nan"), dtype=torch.bfloat16)
        kc[:kv_len] = kstore
        vc[:kv_len] = v
        kc, vc = kc.to(gpu), vc.to(gpu)
        o = torch.empty_like(qg)
        C.call("efm_attention_decode", ctx, ptr(qg), ptr(kc), ptr(vc), ptr(o), 0, ptr(d_len), max_kv, ptr(ws),
               ws.numel(), stream())
        torch.cuda.synchronize()
        outs.append(o)
        caches.append(kc.cpu())
    what = f"{layout} hq={hq} hkv={hkv} hd={hd} L={kv_len}"
    assert torch.isfinite(outs[0].float()).all(), what
    assert_close_bf16(outs[0], ref, what="one-wave splits vs oracle, " + what)
    assert_close_bf16(outs[0], outs[1], what="one-wave splits vs previous kernels, " + what)
    if layout == "rotated_except_newest":
        # the newest row is stored back rotated the same way by both paths; no other row moves
        assert torch.equal(caches[0][: kv_len - 1], kstore[: kv_len - 1])
        assert torch.isnan(caches[0][kv_len:].float()).all()
        assert torch.equal(caches[0][kv_len - 1], caches[1][kv_len - 1])
    else:
        assert torch.equal(caches[0][:kv_len], kstore), "the call must not write the cache"


def test_attention_decode_partials_ignore_stale_rows(gpu):
    """Rows >= L of the cache hold NaN / Inf; the partials + merge path must give the
    same result as a cache that ends at L."""
    torch.manual_seed(9)
    hq, hkv, hd, L, max_kv = 12, 2, 128, 300, 1024
    q = torch.randn(1, hq, hd, dtype=torch.bfloat16, device=gpu)
    k = torch.randn(max_kv, hkv, hd, dtype=torch.bfloat16, device=gpu)
    v = torch.randn(max_kv, hkv, hd, dtype=torch.bfloat16, device=gpu)
    k[L:] = float("inf")
    v[L:] = float("nan")
    ctx = C.make_attention_ctx(hq, hkv, hd)
    d_len = torch.tensor([L], dtype=torch.int32, device=gpu)
    ws = torch.zeros(C.load().efm_attention_decode_workspace_bytes(ctx, max_kv), dtype=torch.uint8, device=gpu)
    o = torch.empty_like(q)
    C.call("efm_attention_decode", ctx, ptr(q), ptr(k), ptr(v), ptr(o), 0, ptr(d_len), max_kv, ptr(ws), ws.numel(),
           stream())
    torch.cuda.synchronize()
    ref = O.attention_decode(q.cpu(), k[:L].cpu(), v[:L].cpu(), L, O.AttnCtx(hq, hkv, hd))
    assert torch.isfinite(o.float()).all()
    assert_close_bf16(o, ref)


@pytest.mark.parametrize("S,base,hq,hkv,hd", [(37, 0, 12, 2, 128), (5, 1000, 14, 2, 64), (300, 16000, 28, 4, 128)])
def test_rope_llama_inplace_matches_oracle(gpu, S, base, hq, hkv, hd):
    """Q in a fused QKV buffer (token stride) and K rows rotated in place at positions
    base + t; one bf16 rounding of the oracle's fp32 rotation."""
    torch.manual_seed(S)
    tot = (hq + 2 * hkv) * hd
    qkv = torch.randn(S, tot, dtype=torch.bfloat16)
    kc = torch.randn(S, hkv, hd, dtype=torch.bfloat16)
    pos = base + torch.arange(S)
    want_q = O.rope_llama(qkv[:, : hq * hd].reshape(S, hq, hd), pos, 1.0e6).to(torch.bfloat16)
    want_k = O.rope_llama(kc, pos, 1.0e6).to(torch.bfloat16)
    qkv_g, kc_g = qkv.to(gpu), kc.to(gpu)
    C.call("efm_rope_llama_inplace", ptr(qkv_g), ptr(kc_g), S, hq, hkv, hd, tot, hkv * hd, base, 1.0e6, 1.0,
           stream())
    torch.cuda.synchronize()
    got = qkv_g.cpu()
    assert_close_bf16(got[:, : hq * hd].reshape(S, hq, hd), want_q, rtol=1e-2, atol=1e-2, what="q")
    assert torch.equal(got[:, hq * hd:], qkv[:, hq * hd:]), "K/V columns of the QKV buffer untouched"
    assert_close_bf16(kc_g, want_k, rtol=1e-2, atol=1e-2, what="k")


@pytest.mark.parametrize("mode,S,base,hq,hkv,hd", [
    ("text", 77, 0, 12, 2, 128), ("text", 300, 513, 28, 4, 128), ("text", 33, 5, 14, 2, 64),
    ("mrope", 70, 0, 16, 2, 128),
])
def test_prefill_rope_write_kv_matches_two_step_and_oracle(gpu, mode, S, base, hq, hkv, hd):
    """One-pass q rotation + rotated K / raw V into the cache rows equals the two-step
    path (K / V copies, then efm_rope_llama_inplace or efm_mrope over the cache rows) bit
    for bit, and the oracle's rotation within one bf16 rounding; cache rows outside
    [base, base + S) and the QKV buffer's K / V columns stay untouched."""
    torch.manual_seed(S + hd)
    kvd, qd = hkv * hd, hq * hd
    tot = qd + 2 * kvd
    rows = base + S + 9
    qkv = torch.randn(S, tot, dtype=torch.bfloat16)
    kc0 = torch.randn(rows, kvd, dtype=torch.bfloat16)
    vc0 = torch.randn(rows, kvd, dtype=torch.bfloat16)
    if mode == "mrope":
        sections = (16, 24, 24)
        pos = (torch.stack([torch.zeros(S, dtype=torch.int32), torch.arange(S, dtype=torch.int32) // 7,
                            torch.arange(S, dtype=torch.int32) % 7]) + 3).contiguous()
        pos_g = pos.to(gpu)
    else:
        sections, pos_g = (hd // 2, 0, 0), None
    # one pass
    q1, k1, v1 = qkv.to(gpu), kc0.to(gpu), vc0.to(gpu)
    C.call("efm_prefill_rope_write_kv", ptr(q1), tot, ptr(k1[base:]), ptr(v1[base:]), kvd, S, hq, hkv, hd,
           ptr(pos_g), S, base if mode == "text" else 0, *sections, 1.0e6, 1.0, stream())
    # two steps
    q2, k2, v2 = qkv.to(gpu), kc0.to(gpu), vc0.to(gpu)
    k2[base:base + S] = q2[:, qd:qd + kvd]
    v2[base:base + S] = q2[:, qd + kvd:]
    if mode == "mrope":
        C.call("efm_mrope", ptr(q2), ptr(k2[base:]), ptr(pos_g), S, S, hq, hkv, hd, tot, kvd, *sections, 1.0e6,
               1.0, stream())
    else:
        C.call("efm_rope_llama_inplace", ptr(q2), ptr(k2[base:]), S, hq, hkv, hd, tot, kvd, base, 1.0e6, 1.0,
               stream())
    torch.cuda.synchronize()
    assert torch.equal(q1, q2) and torch.equal(k1, k2) and torch.equal(v1, v2), "differs from the two-step path"
    assert torch.equal(k1[:base].cpu(), kc0[:base]) and torch.equal(k1[base + S:].cpu(), kc0[base + S:])
    assert torch.equal(q1[:, qd:].cpu(), qkv[:, qd:]), "K / V columns of the QKV buffer untouched"
    if mode == "mrope":
        want_q = O.mrope(qkv[:, :qd].reshape(S, hq, hd), pos, sections, 1.0e6)
        want_k = O.mrope(qkv[:, qd:qd + kvd].reshape(S, hkv, hd), pos, sections, 1.0e6)
    else:
        p = base + torch.arange(S)
        want_q = O.rope_llama(qkv[:, :qd].reshape(S, hq, hd), p, 1.0e6).to(torch.bfloat16)
        want_k = O.rope_llama(qkv[:, qd:qd + kvd].reshape(S, hkv, hd), p, 1.0e6).to(torch.bfloat16)
    assert_close_bf16(q1[:, :qd].reshape(S, hq, hd), want_q, rtol=1e-2, atol=1e-2, what="q")
    assert_close_bf16(k1[base:base + S].reshape(S, hkv, hd), want_k, rtol=1e-2, atol=1e-2, what="k")
    assert torch.equal(v1[base:base + S].cpu(), qkv[:, qd + kvd:]), "V rows copied"


def test_attention_decode_strided_views(gpu):
    """q read from a fused QKV row and K/V from strided views equals contiguous inputs
    (tests/operators/test_attention_prefill.py:167-300)."""
    torch.manual_seed(4)
    hq, hkv, hd, L = 12, 2, 128, 257
    qkv = torch.randn(1, (hq + 2 * hkv) * hd, dtype=torch.bfloat16, device=gpu)
    kv = torch.randn(L, 2, hkv, hd, dtype=torch.bfloat16, device=gpu)  # interleaved K/V rows
    q = qkv[:, : hq * hd].reshape(1, hq, hd)
    k = kv[:, 0]
    v = kv[:, 1]
    ctx = C.make_attention_ctx(hq, hkv, hd, q_stride_n=(hq + 2 * hkv) * hd, q_stride_h=hd,
                               k_stride_n=2 * hkv * hd, k_stride_h=hd, kv_stride_n=2 * hkv * hd, kv_stride_h=hd)
    ws = torch.zeros(C.load().efm_attention_decode_workspace_bytes(ctx, L), dtype=torch.uint8, device=gpu)
    o = torch.empty(1, hq, hd, dtype=torch.bfloat16, device=gpu)
    C.call("efm_attention_decode", ctx, qkv.data_ptr(), kv.data_ptr(), kv[:, 1].data_ptr(), ptr(o), L, None, 0,
           ptr(ws), ws.numel(), stream())
    torch.cuda.synchronize()
    ref, _ = _decode(C.make_attention_ctx(hq, hkv, hd), q.contiguous(), k.contiguous(), v.contiguous(), L)
    assert_close_bf16(o, ref)


def test_attention_decode_rejects_unsupported(gpu):
    ctx = C.make_attention_ctx(10, 2, 128)  # group size 5
    with pytest.raises(C.EfmError) as e:
        C.call("efm_attention_decode", ctx, 1, 1, 1, 1, 1, None, 0, 1, 1 << 20, stream())
    assert e.value.code == C.EFM_ERR_UNSUPPORTED


@pytest.mark.parametrize("batch,hidden", [(1, 896), (1, 1536), (4, 2048), (7, 3584), (512, 1536)])
def test_rms_norm_and_fused_add(gpu, batch, hidden):
    torch.manual_seed(0)
    x = torch.randn(batch, hidden, dtype=torch.bfloat16)
    r = torch.randn(batch, hidden, dtype=torch.bfloat16)
    w = (1 + 0.1 * torch.randn(hidden)).to(torch.bfloat16)
    eps = 1e-6
    xg, rg, wg = x.to(gpu), r.to(gpu), w.to(gpu)
    out = torch.empty_like(xg)
    C.call("efm_rms_norm", batch, hidden, eps, ptr(xg), ptr(wg), ptr(out), stream())
    torch.cuda.synchronize()
    assert_close_bf16(out, O.rms_norm(x, w, eps), what="rms_norm")
    C.call("efm_fused_add_rms_norm", batch, hidden, eps, ptr(xg), ptr(rg), ptr(wg), stream())
    torch.cuda.synchronize()
    ref_out, ref_res = O.fused_add_rms_norm(x, r, w, eps)
    assert torch.equal(rg.cpu(), ref_res), "residual must be bf16(x + r) exactly"
    assert_close_bf16(xg, ref_out, what="fused_add_rms_norm")


@pytest.mark.parametrize("layout", [C.EFM_LAYOUT_UP_GATE, C.EFM_LAYOUT_GATE_UP])
@pytest.mark.parametrize("batch,inter", [(1, 4864), (1, 8960), (5, 11008)])
def test_act_and_mul(gpu, layout, batch, inter):
    torch.manual_seed(0)
    x = torch.randn(batch, 2 * inter, dtype=torch.bfloat16) * 3
    out = torch.empty(batch, inter, dtype=torch.bfloat16, device=gpu)
    xg = x.to(gpu)
    C.call("efm_act_and_mul", batch, inter, layout, ptr(xg), ptr(out), stream())
    torch.cuda.synchronize()
    ref = O.act_and_mul(x, up_first=(layout == C.EFM_LAYOUT_UP_GATE))
    # the north star's per-operator bound (2e-2 / 2e-2; the reference's own test allows
    # atol 6.25e-2, tests/operators/test_fused_gate_up_activation.py:75-79)
    assert_close_bf16(out, ref, rtol=2e-2, atol=2e-2)


@pytest.mark.parametrize("up", [1.0, 0.7421875, -1.3984375, 3.0])
def test_act_and_mul_every_bf16_gate(gpu, up):
    """Every bf16 gate value (signed zeros, infinities and NaNs included) through the
    kernels' silu, against the oracle's g / (1 + exp(-g)): bf16(silu(g) * up) is the same
    bf16 value except for a handful of 1-ulp roundings and, for g in (-88.7, -87.3), results
    under 1e-35 that come out as zeros of the same sign."""
    g = torch.arange(65536, dtype=torch.int32).to(torch.int16).view(torch.bfloat16)
    n = g.numel()
    x = torch.cat([torch.full((n,), up, dtype=torch.bfloat16), g]).reshape(1, 2 * n)
    xg = x.to(gpu)
    out = torch.empty(1, n, dtype=torch.bfloat16, device=gpu)
    C.call("efm_act_and_mul", 1, n, C.EFM_LAYOUT_UP_GATE, ptr(xg), ptr(out), stream())
    torch.cuda.synchronize()
    o, ref = out.cpu().flatten(), O.act_and_mul(x, up_first=True).flatten()
    of, rf = o.float(), ref.float()
    same = (o.view(torch.int16) == ref.view(torch.int16)) | (torch.isnan(of) & torch.isnan(rf))
    bad = (~same).nonzero().flatten()
    tiny = (rf[bad].abs() < 1e-35) & (of[bad] == 0) & (torch.signbit(of[bad]) == torch.signbit(rf[bad]))
    assert tiny.sum() <= 3 and bool(((g[bad].float() > -88.75) & (g[bad].float() < -87.25))[tiny].all())
    near = bad[~tiny]
    assert near.numel() <= 4, [(float(g[i]), float(o[i]), float(ref[i])) for i in near[:8]]
    assert bool(((o.view(torch.int16)[near].int() - ref.view(torch.int16)[near].int()).abs() == 1).all())
    assert torch.signbit(of[g.float() == 0]).tolist() == torch.signbit(rf[g.float() == 0]).tolist()


LINEAR_CASES = [
    pytest.param(1536, 2048, True, id="1p5b_qkv"),
    pytest.param(1536, 1536, False, id="1p5b_o"),
    pytest.param(8960, 1536, False, id="1p5b_down"),
    pytest.param(896, 1152, True, id="0p5b_qkv"),
    pytest.param(4864, 896, False, id="0p5b_down"),
    pytest.param(18944, 3584, False, id="7b_down"),
    pytest.param(3584, 4608, True, id="7b_qkv"),
]


@pytest.mark.parametrize("k,n,bias", LINEAR_CASES)
@pytest.mark.parametrize("m", [1, 3, 64, 512])
def test_linear(gpu, k, n, bias, m):
    torch.manual_seed(0)
    x = torch.randn(m, k, dtype=torch.bfloat16)
    w = (torch.randn(n, k) * 0.02).to(torch.bfloat16)
    b = (torch.randn(n) * 0.02).to(torch.bfloat16) if bias else None
    y = torch.empty(m, n, dtype=torch.bfloat16, device=gpu)
    xg, wg, bg = x.to(gpu), w.to(gpu), (b.to(gpu) if bias else None)
    C.call("efm_linear", m, k, n, ptr(xg), ptr(wg), ptr(bg), ptr(y), C.EFM_DTYPE_BF16, stream())
    torch.cuda.synchronize()
    assert_close_bf16(y, O.linear(x, w, b), what=f"linear m={m}")


@pytest.mark.parametrize("m", [1, 17])
def test_linear_fp32_logits(gpu, m):
    torch.manual_seed(0)
    k, n = 1536, 151936
    x = torch.randn(m, k, dtype=torch.bfloat16)
    w = (torch.randn(n, k) * 0.02).to(torch.bfloat16)
    y = torch.empty(m, n, dtype=torch.float32, device=gpu)
    xg, wg = x.to(gpu), w.to(gpu)
    C.call("efm_linear", m, k, n, ptr(xg), ptr(wg), None, ptr(y), C.EFM_DTYPE_F32, stream())
    torch.cuda.synchronize()
    torch.testing.assert_close(y.cpu(), O.linear(x, w, out_f32=True), rtol=1e-4, atol=1e-4)


@pytest.mark.parametrize("m,k,n,bias,kind", [
    pytest.param(4100, 1024, 12345, True, "bf16", id="ragged_bias"),
    pytest.param(6144, 1536, 8192, False, "bf16", id="1p5b_like"),
    pytest.param(4096, 2048, 11008, False, "swiglu", id="vl3b_gate_up"),
    pytest.param(300, 1536, 151936, False, "f32", id="logits_f32"),
])
def test_gemm_large_shapes_row_sample_vs_oracle(gpu, m, k, n, bias, kind):
    """Large and ragged prefill shapes (partial edge tiles in M and N) against the oracle
    on a row sample."""
    torch.manual_seed(m + n)
    x = torch.randn(m, k, dtype=torch.bfloat16, device=gpu)
    nw = 2 * n if kind == "swiglu" else n
    w = (torch.randn(nw, k, device=gpu) * 0.05).to(torch.bfloat16)
    b = (torch.randn(n, device=gpu) * 0.05).to(torch.bfloat16) if bias else None
    if kind == "swiglu":
        y = torch.empty(m, n, dtype=torch.bfloat16, device=gpu)
        C.call("efm_fused_gate_up_swiglu", m, k, n, ptr(x), ptr(w), ptr(y), stream())
    else:
        dt = torch.float32 if kind == "f32" else torch.bfloat16
        y = torch.empty(m, n, dtype=dt, device=gpu)
        C.call("efm_linear", m, k, n, ptr(x), ptr(w), ptr(b), ptr(y),
               C.EFM_DTYPE_F32 if kind == "f32" else C.EFM_DTYPE_BF16, stream())
    torch.cuda.synchronize()
    rows = torch.tensor([0, m // 2, m - 1])
    xs = x[rows].cpu()
    if kind == "swiglu":
        assert_close_bf16(y[rows], O.gate_up_swiglu(xs, w.cpu()), rtol=2e-2, atol=2e-2)
    elif kind == "f32":
        torch.testing.assert_close(y[rows].cpu(), O.linear(xs, w.cpu(), out_f32=True), rtol=1e-4, atol=1e-4)
    else:
        assert_close_bf16(y[rows], O.linear(xs, w.cpu(), None if b is None else b.cpu()))


@pytest.mark.parametrize("hidden,inter", [(896, 4864), (1536, 8960), (3584, 18944)])
@pytest.mark.parametrize("m", [1, 5, 300])
def test_fused_gate_up_swiglu(gpu, hidden, inter, m):
    torch.manual_seed(0)
    x = torch.randn(m, hidden, dtype=torch.bfloat16)
    w = (torch.randn(2 * inter, hidden) * 0.05).to(torch.bfloat16)
    out = torch.empty(m, inter, dtype=torch.bfloat16, device=gpu)
    xg, wg = x.to(gpu), w.to(gpu)
    C.call("efm_fused_gate_up_swiglu", m, hidden, inter, ptr(xg), ptr(wg), ptr(out), stream())
    torch.cuda.synchronize()
    assert_close_bf16(out, O.gate_up_swiglu(x, w), rtol=2e-2, atol=2e-2)


def _top1_ref_ok(logits: torch.Tensor, tok: int) -> bool:
    """GPU top-1 equals the oracle argmax, or the two differ by less than the fp32
    accumulation-order noise (near tie)."""
    ref = int(O.argmax_lowest(logits.unsqueeze(0))[0])
    if tok == ref:
        return True
    return abs(float(logits[tok]) - float(logits[ref])) < 1e-4 * max(1.0, abs(float(logits[ref])))


@pytest.mark.parametrize("hidden,vocab", [(896, 151936), (1536, 151936), (3584, 152064)])
def test_lm_head_top1(gpu, hidden, vocab):
    torch.manual_seed(0)
    x = torch.randn(1, hidden, dtype=torch.bfloat16)
    w = (torch.randn(vocab, hidden) * 0.02).to(torch.bfloat16)
    ws = torch.zeros(C.load().efm_lm_head_top1_workspace_bytes(vocab), dtype=torch.uint8, device=gpu)
    tok = torch.full((1,), -1, dtype=torch.int32, device=gpu)
    xg, wg = x.to(gpu), w.to(gpu)
    for _ in range(3):  # counter must reset itself between calls
        C.call("efm_lm_head_top1", hidden, vocab, ptr(xg), ptr(wg), ptr(tok), ptr(ws), ws.numel(), stream())
        torch.cuda.synchronize()
        assert _top1_ref_ok(O.linear(x, w, out_f32=True)[0], int(tok.item()))


def test_lm_head_top1_ties_pick_lowest_index(gpu):
    """Duplicate the winning row at a higher and a lower index: the lowest wins
    (src/layers/linear.cu:155-160)."""
    torch.manual_seed(5)
    hidden, vocab = 1536, 151936
    x = torch.randn(1, hidden, dtype=torch.bfloat16)
    w = (torch.randn(vocab, hidden) * 0.02).to(torch.bfloat16)
    w[99_000] = x[0] * 0.1
    w[150_000] = w[99_000]
    w[1234] = w[99_000]
    ws = torch.zeros(C.load().efm_lm_head_top1_workspace_bytes(vocab), dtype=torch.uint8, device=gpu)
    tok = torch.full((1,), -1, dtype=torch.int32, device=gpu)
    xg, wg = x.to(gpu), w.to(gpu)
    C.call("efm_lm_head_top1", hidden, vocab, ptr(xg), ptr(wg), ptr(tok), ptr(ws), ws.numel(), stream())
    torch.cuda.synchronize()
    assert int(tok.item()) == 1234


def test_lm_head_top1_negative_scores_edges_and_clean_workspace(gpu):
    """All scores negative (the order-preserving key must rank negative values by
    magnitude), winner in the last row, then tied with row 0 (row 0 wins); every launch
    leaves the workspace zeroed for the next."""
    torch.manual_seed(6)
    hidden, vocab = 1536, 151936
    x = torch.rand(1, hidden).add(0.5).to(torch.bfloat16)
    w = -(torch.rand(vocab, hidden) * 0.02 + 0.01)
    w[vocab - 1] *= 0.25
    w = w.to(torch.bfloat16)
    ws = torch.zeros(C.load().efm_lm_head_top1_workspace_bytes(vocab), dtype=torch.uint8, device=gpu)
    tok = torch.full((1,), -1, dtype=torch.int32, device=gpu)
    xg, wg = x.to(gpu), w.to(gpu)
    ref = O.linear(x, w, out_f32=True)[0]
    assert float(ref.max()) < 0
    for expect in (vocab - 1, 0):
        if expect == 0:
            wg[0] = wg[vocab - 1]
        C.call("efm_lm_head_top1", hidden, vocab, ptr(xg), ptr(wg), ptr(tok), ptr(ws), ws.numel(), stream())
        torch.cuda.synchronize()
        assert int(tok.item()) == expect
        assert int(ws.count_nonzero()) == 0


@pytest.mark.parametrize("kind", ["bf16", "swiglu"])
def test_gemm_tile_shapes_agree_bit_exact(gpu, kind):
    """The kernel and tile shape follow M: 100 rows run 64 x 64 (SwiGLU 64 x 128), 300
    rows 128 x 64 (SwiGLU 128 x 128), 1344 rows 128 x 128 (many tiles per XCD: the
    grouped tile order) and 6144 rows the 256 x 256 wide kernel. Every kernel sums each
    output over K in the same order, so the first 100 rows must agree bit for bit across
    all launches (and with the oracle on a sample)."""
    torch.manual_seed(17)
    k, n = 1024, 8192
    x = torch.randn(6144, k, dtype=torch.bfloat16, device=gpu)
    nw = 2 * n if kind == "swiglu" else n
    w = (torch.randn(nw, k, device=gpu) * 0.05).to(torch.bfloat16)
    b = (torch.randn(n, device=gpu) * 0.05).to(torch.bfloat16) if kind == "bf16" else None
    heads = []
    for m in (100, 300, 1344, 6144):
        y = torch.empty(m, n, dtype=torch.bfloat16, device=gpu)
        if kind == "swiglu":
            C.call("efm_fused_gate_up_swiglu", m, k, n, ptr(x), ptr(w), ptr(y), stream())
        else:
            C.call("efm_linear", m, k, n, ptr(x), ptr(w), ptr(b), ptr(y), C.EFM_DTYPE_BF16, stream())
        torch.cuda.synchronize()
        heads.append(y[:100].clone())
    for m, h in zip((300, 1344, 6144), heads[1:]):
        assert torch.equal(h, heads[0]), f"{kind}: rows of the M={m} launch differ from the M=100 launch"
    rows = torch.tensor([0, 57, 99])
    xs = x[rows].cpu()
    if kind == "swiglu":
        assert_close_bf16(heads[0][rows], O.gate_up_swiglu(xs, w.cpu()), rtol=2e-2, atol=2e-2)
    else:
        assert_close_bf16(heads[0][rows], O.linear(xs, w.cpu(), b.cpu()))


@pytest.mark.parametrize("m,k,n,kind", [
    pytest.param(4096, 1024, 3072, "bf16", id="aligned"),
    pytest.param(1000, 2048, 1000, "bias", id="ragged_m_n"),
    pytest.param(777, 1536, 2400, "swiglu", id="ragged_swiglu"),
    pytest.param(513, 3584, 4608, "f32", id="f32_bias"),
    pytest.param(512, 1536, 8960, "swiglu", id="c2_gate_up"),
])
def test_gemm_wide_kernel_matches_narrow_bit_exact(gpu, knob, m, k, n, kind):
    """The 256 x 256 wide kernel (EFM_KNOB_GEMM_TILE 2) and its 192 x 256 tiles (knob 3:
    12 A and 16 B blocks per stage over 8 waves) against the 128 x 128 family (knob 1) on
    aligned and ragged shapes and every epilogue: bit-identical outputs (all sum keys 16
    at a time in increasing order), and a row sample against the oracle."""
    torch.manual_seed(m + n)
    x = torch.randn(m, k, dtype=torch.bfloat16, device=gpu)
    nw = 2 * n if kind == "swiglu" else n
    w = (torch.randn(nw, k, device=gpu) * 0.05).to(torch.bfloat16)
    b = (torch.randn(n, device=gpu) * 0.05).to(torch.bfloat16) if kind in ("bias", "f32") else None
    odt = torch.float32 if kind == "f32" else torch.bfloat16
    outs = []
    for path in (1, 2, 3):
        knob(C.EFM_KNOB_GEMM_TILE, path)
        y = torch.full((m, n), float("nan"), dtype=odt, device=gpu)
        if kind == "swiglu":
            C.call("efm_fused_gate_up_swiglu", m, k, n, ptr(x), ptr(w), ptr(y), stream())
        else:
            cd = C.EFM_DTYPE_F32 if kind == "f32" else C.EFM_DTYPE_BF16
            C.call("efm_linear", m, k, n, ptr(x), ptr(w), ptr(b), ptr(y), cd, stream())
        torch.cuda.synchronize()
        outs.append(y)
    for path, y in zip((2, 3), outs[1:]):
        assert not torch.isnan(y).any(), f"wide kernel (knob {path}) left outputs unwritten"
        assert torch.equal(outs[0], y), f"{kind}: wide (knob {path}) and narrow kernels differ"
    rows = torch.tensor([0, m // 2, m - 1])
    xs = x[rows].cpu()
    if kind == "swiglu":
        assert_close_bf16(outs[1][rows], O.gate_up_swiglu(xs, w.cpu()), rtol=2e-2, atol=2e-2)
    elif kind == "f32":
        ref = O.linear(xs, w.cpu(), b.cpu(), out_f32=True)
        torch.testing.assert_close(outs[1][rows].cpu(), ref, rtol=1e-3, atol=1e-3)
    else:
        assert_close_bf16(outs[1][rows], O.linear(xs, w.cpu(), b.cpu() if b is not None else None))


@pytest.mark.parametrize("m,k,n,kind", [
    pytest.param(512, 8960, 1536, "bf16", id="c2_down"),
    pytest.param(300, 18944, 3584, "bf16", id="7b_down"),
    pytest.param(300, 4096, 1000, "bias", id="ragged_bias"),
    pytest.param(200, 8192, 2048, "f32", id="f32"),
    pytest.param(1024, 8960, 1536, "bf16", id="shallow_split"),
])
def test_linear_split_k_matches_unsplit_and_oracle(gpu, m, k, n, kind):
    """efm_linear_ws splits K for these under-filled, long-K shapes: its result equals
    efm_linear to fp32 rounding, is deterministic, matches the oracle on a row sample, and
    with too small a workspace the call is exactly efm_linear."""
    torch.manual_seed(m + k)
    need = C.load().efm_linear_workspace_bytes(m, k, n)
    assert need > 0
    x = torch.randn(m, k, dtype=torch.bfloat16, device=gpu)
    w = (torch.randn(n, k, device=gpu) * 0.02).to(torch.bfloat16)
    b = (torch.randn(n, device=gpu) * 0.05).to(torch.bfloat16) if kind == "bias" else None
    f32 = kind == "f32"
    dt, cd = (torch.float32, C.EFM_DTYPE_F32) if f32 else (torch.bfloat16, C.EFM_DTYPE_BF16)
    ws = torch.full((need,), 0x7f, dtype=torch.uint8, device=gpu)
    outs = []
    for wsz in (need, need, 64):
        y = torch.empty(m, n, dtype=dt, device=gpu)
        C.call("efm_linear_ws", m, k, n, ptr(x), ptr(w), ptr(b), ptr(y), cd, ptr(ws), wsz, stream())
        torch.cuda.synchronize()
        outs.append(y)
    ref = torch.empty(m, n, dtype=dt, device=gpu)
    C.call("efm_linear", m, k, n, ptr(x), ptr(w), ptr(b), ptr(ref), cd, stream())
    torch.cuda.synchronize()
    assert torch.equal(outs[0], outs[1]), "split-K is not deterministic"
    assert torch.equal(outs[2], ref), "too small a workspace must run the unsplit GEMM"
    if f32:
        torch.testing.assert_close(outs[0], ref, rtol=1e-5, atol=1e-4)
    else:
        diff = (outs[0].float() - ref.float()).abs()
        assert float(diff.max()) <= float(ref.float().abs().max()) * 2 ** -7, "split-K differs beyond one bf16 ulp"
    rows = torch.tensor([0, m // 2, m - 1])
    exp = O.linear(x[rows].cpu(), w.cpu(), None if b is None else b.cpu(), out_f32=f32)
    if f32:
        torch.testing.assert_close(outs[0][rows].cpu(), exp, rtol=1e-4, atol=1e-4)
    else:
        assert_close_bf16(outs[0][rows], exp)


def test_gemm_long_k_tiles_agree_bit_exact(gpu):
    """K = 11008 (the VL-3B down projection) at three M: 100 rows run 64 x 64 tiles, 1344
    rows (176 tiles of 128 x 128, at most one per CU) 128 x 128 tiles over a 4-deep ring
    with one workgroup per CU, 2300 rows 128 x 64 tiles over a 3-deep ring. All sum each
    output over K in the same order: the first 100 rows agree bit for bit, and a row
    sample of each launch matches the oracle."""
    torch.manual_seed(29)
    k, n = 11008, 2048
    x = torch.randn(2300, k, dtype=torch.bfloat16, device=gpu)
    w = (torch.randn(n, k, device=gpu) * 0.02).to(torch.bfloat16)
    b = (torch.randn(n, device=gpu) * 0.05).to(torch.bfloat16)
    outs = {}
    for m in (100, 1344, 2300):
        y = torch.full((m, n), float("nan"), dtype=torch.bfloat16, device=gpu)
        C.call("efm_linear", m, k, n, ptr(x), ptr(w), ptr(b), ptr(y), C.EFM_DTYPE_BF16, stream())
        torch.cuda.synchronize()
        assert not torch.isnan(y).any(), f"M={m}: outputs left unwritten"
        outs[m] = y
    for m in (1344, 2300):
        assert torch.equal(outs[m][:100], outs[100]), f"rows of the M={m} launch differ from the M=100 launch"
        rows = torch.tensor([0, m // 2, m - 1])
        assert_close_bf16(outs[m][rows], O.linear(x[rows].cpu(), w.cpu(), b.cpu()))


def test_linear_workspace_bytes_zero_without_split(gpu):
    lib = C.load()
    assert lib.efm_linear_workspace_bytes(1, 8960, 1536) == 0          # GEMV
    assert lib.efm_linear_workspace_bytes(16384, 18944, 3584) == 0     # enough tiles
    assert lib.efm_linear_workspace_bytes(512, 1536, 1536) == 0        # short K
    assert lib.efm_linear_workspace_bytes(1344, 11008, 2048) == 0      # 176 tiles: no gain
    assert lib.efm_linear_workspace_bytes(512, 8960, 1536) > 0


@pytest.mark.parametrize("m,k,n,bias", [
    pytest.param(1344, 2048, 2560, True, id="c3_qkv"),
    pytest.param(1344, 11008, 2048, False, id="c3_down"),
    pytest.param(512, 8960, 1536, False, id="c2_down"),
    pytest.param(77, 1536, 2048, True, id="ragged_m"),
    pytest.param(2, 896, 1000, False, id="m2"),
])
def test_linear_workspace_path_matches_oracle_and_repeats(gpu, m, k, n, bias):
    """The prefill GEMM with its workspace (split-K where the plan asks for it) and without
    one: both match the oracle on a row sample, each repeats bit for bit, and the two agree
    to bf16 rounding (the split sums K in another order)."""
    torch.manual_seed(m + n)
    x = torch.randn(m, k, dtype=torch.bfloat16, device=gpu)
    w = (torch.randn(n, k, device=gpu) * 0.02).to(torch.bfloat16)
    b = (torch.randn(n, device=gpu) * 0.05).to(torch.bfloat16) if bias else None
    need = C.load().efm_linear_workspace_bytes(m, k, n)
    ws = torch.full((max(need, 256),), 0x7f, dtype=torch.uint8, device=gpu)
    outs = []
    for use_ws in (True, True, False, False):
        y = torch.full((m, n), float("nan"), dtype=torch.bfloat16, device=gpu)
        if use_ws:
            C.call("efm_linear_ws", m, k, n, ptr(x), ptr(w), ptr(b), ptr(y), C.EFM_DTYPE_BF16, ptr(ws), need,
                   stream())
        else:
            C.call("efm_linear", m, k, n, ptr(x), ptr(w), ptr(b), ptr(y), C.EFM_DTYPE_BF16, stream())
        torch.cuda.synchronize()
        outs.append(y)
    assert torch.equal(outs[0], outs[1]) and torch.equal(outs[2], outs[3]), "GEMM is not deterministic"
    scale = float(outs[2].float().abs().max())
    assert torch.isfinite(outs[0].float()).all()
    assert float((outs[0].float() - outs[2].float()).abs().max()) <= scale * 2 ** -7
    rows = torch.tensor([0, m // 2, m - 1])
    exp = O.linear(x[rows].cpu(), w.cpu(), None if b is None else b.cpu())
    assert_close_bf16(outs[0][rows], exp)
    assert_close_bf16(outs[2][rows], exp)


def test_linear_workspace_plan_ignores_spare_capacity(gpu):
    """A caller whose grow-only scratch is larger than a shape needs gets the same bits as
    one passing exactly the shape's figure: the split-K plan depends on the shape alone."""
    torch.manual_seed(3)
    m, k, n = 512, 8960, 1536
    x = torch.randn(m, k, dtype=torch.bfloat16, device=gpu)
    w = (torch.randn(n, k, device=gpu) * 0.02).to(torch.bfloat16)
    need = C.load().efm_linear_workspace_bytes(m, k, n)
    big = 3 * need
    assert need > 0
    ws = torch.zeros(big, dtype=torch.uint8, device=gpu)
    a = torch.empty(m, n, dtype=torch.bfloat16, device=gpu)
    b = torch.empty_like(a)
    C.call("efm_linear_ws", m, k, n, ptr(x), ptr(w), None, ptr(a), C.EFM_DTYPE_BF16, ptr(ws), need, stream())
    C.call("efm_linear_ws", m, k, n, ptr(x), ptr(w), None, ptr(b), C.EFM_DTYPE_BF16, ptr(ws), big, stream())
    torch.cuda.synchronize()
    assert torch.equal(a, b)


def test_linear_unaligned_output(gpu):
    """An output pointer that is only 2-byte aligned is written correctly."""
    torch.manual_seed(8)
    m, k, n = 64, 1024, 1000
    x = torch.randn(m, k, dtype=torch.bfloat16, device=gpu)
    w = (torch.randn(n, k, device=gpu) * 0.02).to(torch.bfloat16)
    buf = torch.zeros(m * n + 8, dtype=torch.bfloat16, device=gpu)
    out = buf[1:1 + m * n]                       # 2-byte offset
    assert out.data_ptr() % 16 != 0
    C.call("efm_linear", m, k, n, ptr(x), ptr(w), None, ptr(out), C.EFM_DTYPE_BF16, stream())
    aligned = torch.empty(m, n, dtype=torch.bfloat16, device=gpu)
    C.call("efm_linear", m, k, n, ptr(x), ptr(w), None, ptr(aligned), C.EFM_DTYPE_BF16, stream())
    torch.cuda.synchronize()
    assert torch.equal(out.reshape(m, n), aligned)
    assert float(buf[0]) == 0.0 and float(buf[1 + m * n]) == 0.0
    assert_close_bf16(aligned[:3], O.linear(x[:3].cpu(), w.cpu()))


def test_linear_under_graph_capture(gpu):
    """A prefill GEMM captured into a HIP graph: every replay equals the eager call bit for
    bit, with eager calls between replays."""
    torch.manual_seed(5)
    m, k, n = 96, 1536, 2048
    x = torch.randn(m, k, dtype=torch.bfloat16, device=gpu)
    w = (torch.randn(n, k, device=gpu) * 0.02).to(torch.bfloat16)
    b = (torch.randn(n, device=gpu) * 0.05).to(torch.bfloat16)
    own = torch.empty(m, n, dtype=torch.bfloat16, device=gpu)
    C.call("efm_linear", m, k, n, ptr(x), ptr(w), ptr(b), ptr(own), C.EFM_DTYPE_BF16, stream())
    torch.cuda.synchronize()
    y = torch.empty(m, n, dtype=torch.bfloat16, device=gpu)
    st = torch.cuda.Stream()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=st, capture_error_mode="thread_local"):
        C.call("efm_linear", m, k, n, ptr(x), ptr(w), ptr(b), ptr(y), C.EFM_DTYPE_BF16, st.cuda_stream)
    for rep in range(3):
        y.fill_(float("nan"))
        eager = torch.empty(m, n, dtype=torch.bfloat16, device=gpu)
        C.call("efm_linear", m, k, n, ptr(x), ptr(w), ptr(b), ptr(eager), C.EFM_DTYPE_BF16, stream())
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(y, own), f"replay {rep}"
        assert torch.equal(eager, own)


@pytest.mark.parametrize("m,hidden,inter", [(1344, 2048, 11008), (512, 1536, 8960), (33, 896, 4864)])
def test_gate_up_swiglu_ws_is_fused_kernel(gpu, m, hidden, inter):
    """efm_fused_gate_up_swiglu_ws needs no workspace and equals efm_fused_gate_up_swiglu bit
    for bit; it agrees with efm_linear into [m, 2 inter] + efm_act_and_mul (the reference's
    two-stage path) to bf16 rounding, and with the oracle on sampled rows."""
    torch.manual_seed(m)
    x = torch.randn(m, hidden, dtype=torch.bfloat16, device=gpu)
    w = (torch.randn(2 * inter, hidden, device=gpu) * 0.03).to(torch.bfloat16)
    assert C.load().efm_fused_gate_up_swiglu_workspace_bytes(m, hidden, inter) == 0
    out = torch.empty(m, inter, dtype=torch.bfloat16, device=gpu)
    C.call("efm_fused_gate_up_swiglu_ws", m, hidden, inter, ptr(x), ptr(w), ptr(out), None, 0, stream())
    fused = torch.empty_like(out)
    C.call("efm_fused_gate_up_swiglu", m, hidden, inter, ptr(x), ptr(w), ptr(fused), stream())
    gu = torch.empty(m, 2 * inter, dtype=torch.bfloat16, device=gpu)
    C.call("efm_linear", m, hidden, 2 * inter, ptr(x), ptr(w), None, ptr(gu), C.EFM_DTYPE_BF16, stream())
    two = torch.empty_like(out)
    C.call("efm_act_and_mul", m, inter, C.EFM_LAYOUT_UP_GATE, ptr(gu), ptr(two), stream())
    torch.cuda.synchronize()
    assert torch.equal(out, fused)
    diff = (two.float() - fused.float()).abs()
    assert float(diff.max()) <= float(fused.float().abs().max()) * 2 ** -6
    rows = torch.tensor([0, m - 1])
    assert_close_bf16(out[rows], O.gate_up_swiglu(x[rows].cpu(), w.cpu()), rtol=2e-2, atol=2e-2)


def test_sampler_greedy_ties(gpu):
    torch.manual_seed(0)
    rows, vocab = 4, 151936
    logits = torch.randn(rows, vocab)
    logits[0, 17] = logits[0, 9000] = 50.0
    logits[1, vocab - 1] = 60.0
    logits[2, :] = 1.0
    logits[3, 123456] = 7.0
    logits[3, 123455] = 7.0
    ws = torch.zeros(C.load().efm_sampler_greedy_workspace_bytes(rows, vocab), dtype=torch.uint8, device=gpu)
    out = torch.empty(rows, dtype=torch.int32, device=gpu)
    lg = logits.to(gpu)
    C.call("efm_sampler_greedy", rows, vocab, ptr(lg), ptr(out), ptr(ws), ws.numel(), stream())
    torch.cuda.synchronize()
    assert out.cpu().tolist() == O.argmax_lowest(logits).tolist() == [17, vocab - 1, 0, 123455]


def test_embedding_lookup_with_insertion(gpu):
    torch.manual_seed(0)
    V, H = 1000, 1536
    table = torch.randn(V, H).to(torch.bfloat16)
    custom = torch.randn(5, H).to(torch.bfloat16)
    ids = torch.tensor([3, 999, -1, 1000, 700, 701, 704, 705, 0], dtype=torch.int32)
    out = torch.empty(ids.numel(), H, dtype=torch.bfloat16, device=gpu)
    idg, tg, cg = ids.to(gpu), table.to(gpu), custom.to(gpu)
    C.call("efm_embedding_lookup", ids.numel(), H, V, ptr(idg), ptr(tg), ptr(cg), 5, 700, ptr(out), stream())
    torch.cuda.synchronize()
    assert torch.equal(out.cpu(), O.embedding(ids, table, custom, 700))


def test_decode_runtime_kernels(gpu):
    kdim, vdim, rows = 256, 256, 10
    kc = torch.zeros(rows, kdim, dtype=torch.bfloat16, device=gpu)
    vc = torch.zeros(rows, vdim, dtype=torch.bfloat16, device=gpu)
    ks = torch.randn(kdim).to(torch.bfloat16).to(gpu)
    vs = torch.randn(vdim).to(torch.bfloat16).to(gpu)
    d_len = torch.tensor([4], dtype=torch.int32, device=gpu)
    C.call("efm_copy_decode_kv_cache_slots", ptr(ks), ptr(vs), ptr(kc), ptr(vc), kdim, vdim, ptr(d_len), stream())
    sampled = torch.tensor([42], dtype=torch.int32, device=gpu)
    resp = torch.zeros(3, dtype=torch.int32, device=gpu)
    C.call("efm_finalize_decode_token", ptr(sampled), resp[1:].data_ptr(), ptr(d_len), stream())
    trip = torch.tensor([5, 6, 7], dtype=torch.int32, device=gpu)
    C.call("efm_increment_int32_triplet", ptr(trip), stream())
    torch.cuda.synchronize()
    assert torch.equal(kc[3], ks) and torch.equal(vc[3], vs)
    assert kc[:3].abs().sum() == 0 and kc[4:].abs().sum() == 0
    assert resp.cpu().tolist() == [0, 42, 0] and int(d_len.item()) == 5
    assert trip.cpu().tolist() == [6, 7, 8]


@pytest.mark.parametrize("hidden,hq,hkv,hd", [(1536, 12, 2, 128), (896, 14, 2, 64), (3584, 28, 4, 128)])
@pytest.mark.parametrize("layer0", [True, False])
def test_decode_norm_qkv_matches_unfused(gpu, hidden, hq, hkv, hd, layer0):
    torch.manual_seed(0)
    eps = 1e-6
    qd, kvd = hq * hd, hkv * hd
    h = torch.randn(1, hidden, dtype=torch.bfloat16)
    r = torch.randn(1, hidden, dtype=torch.bfloat16)
    nw = (1 + 0.1 * torch.randn(hidden)).to(torch.bfloat16)
    W = (torch.randn(qd + 2 * kvd, hidden) * 0.02).to(torch.bfloat16)
    b = (torch.randn(qd + 2 * kvd) * 0.02).to(torch.bfloat16)
    rows = 20
    kc = torch.zeros(rows, kvd, dtype=torch.bfloat16, device=gpu)
    vc = torch.zeros(rows, kvd, dtype=torch.bfloat16, device=gpu)
    d_len = torch.tensor([13], dtype=torch.int32, device=gpu)
    q_out = torch.empty(1, qd, dtype=torch.bfloat16, device=gpu)
    r_out = torch.empty(1, hidden, dtype=torch.bfloat16, device=gpu)
    hg, rg, nwg, Wg, bg = h.to(gpu), r.to(gpu), nw.to(gpu), W.to(gpu), b.to(gpu)
    C.call("efm_decode_norm_qkv", hidden, qd, kvd, eps, ptr(hg), None if layer0 else ptr(rg), ptr(r_out), ptr(nwg),
           ptr(Wg), ptr(bg), ptr(q_out), ptr(kc), ptr(vc), ptr(d_len), stream())
    torch.cuda.synchronize()
    if layer0:
        n, res = O.rms_norm(h, nw, eps), h
    else:
        n, res = O.fused_add_rms_norm(h, r, nw, eps)
    qkv = O.linear(n, W, b)
    assert torch.equal(r_out.cpu(), res)
    assert_close_bf16(q_out, qkv[:, :qd], what="q")
    assert_close_bf16(kc[12:13], qkv[:, qd:qd + kvd], what="k slot")
    assert_close_bf16(vc[12:13], qkv[:, qd + kvd:], what="v slot")
    assert kc[:12].abs().sum() == 0 and kc[13:].abs().sum() == 0


@pytest.mark.parametrize("hidden,hq,hkv,hd", [(1536, 12, 2, 128), (896, 14, 2, 64), (3584, 28, 4, 128)])
@pytest.mark.parametrize("layer0", [True, False])
@pytest.mark.parametrize("pos_off", [0, 5])
def test_decode_norm_qkv_rope_matches_oracle(gpu, hidden, hq, hkv, hd, layer0, pos_off):
    """efm_decode_norm_qkv_rope: the projection of efm_decode_norm_qkv with q and the new
    key rotated at position L - 1 (+ offset) in the epilogue: q_out and the K slot equal
    the oracle's rope_llama of the bf16 projection (one bf16 rounding), V and the residual
    are exact; no other cache row is written. Then decode attention with pos NONE over
    that cache equals the oracle's RoPE-on-read attention over the un-rotated keys."""
    torch.manual_seed(1 + hd)
    eps, theta, L = 1e-6, 1.0e6, 300
    qd, kvd = hq * hd, hkv * hd
    h = torch.randn(1, hidden, dtype=torch.bfloat16)
    r = torch.randn(1, hidden, dtype=torch.bfloat16)
    nw = (1 + 0.1 * torch.randn(hidden)).to(torch.bfloat16)
    W = (torch.randn(qd + 2 * kvd, hidden) * 0.02).to(torch.bfloat16)
    b = (torch.randn(qd + 2 * kvd) * 0.02).to(torch.bfloat16)
    k_prev = torch.randn(L - 1, hkv, hd, dtype=torch.bfloat16)
    v_prev = torch.randn(L - 1, hkv, hd, dtype=torch.bfloat16)
    rows = L + 20
    kc = torch.zeros(rows, kvd, dtype=torch.bfloat16)
    vc = torch.zeros(rows, kvd, dtype=torch.bfloat16)
    kc[: L - 1] = O.rope_llama(k_prev, torch.arange(L - 1) + pos_off, theta).to(torch.bfloat16).reshape(L - 1, kvd)
    vc[: L - 1] = v_prev.reshape(L - 1, kvd)
    kc, vc = kc.to(gpu), vc.to(gpu)
    d_len = torch.tensor([L], dtype=torch.int32, device=gpu)
    q_out = torch.empty(1, qd, dtype=torch.bfloat16, device=gpu)
    r_out = torch.empty(1, hidden, dtype=torch.bfloat16, device=gpu)
    ctx = C.make_attention_ctx(hq, hkv, hd, rope_theta=theta, q_rope_pos_offset=pos_off, k_rope_pos_offset=pos_off)
    hg, rg, nwg, Wg, bg = h.to(gpu), r.to(gpu), nw.to(gpu), W.to(gpu), b.to(gpu)
    C.call("efm_decode_norm_qkv_rope", ctx, hidden, eps, ptr(hg), None if layer0 else ptr(rg), ptr(r_out), ptr(nwg),
           ptr(Wg), ptr(bg), ptr(q_out), ptr(kc), ptr(vc), ptr(d_len), stream())
    torch.cuda.synchronize()
    if layer0:
        n, res = O.rms_norm(h, nw, eps), h
    else:
        n, res = O.fused_add_rms_norm(h, r, nw, eps)
    qkv = O.linear(n, W, b)
    pos = torch.tensor([L - 1 + pos_off])
    q_ref = O.rope_llama(qkv[:, :qd].reshape(1, hq, hd), pos, theta).to(torch.bfloat16).reshape(1, qd)
    k_new = qkv[:, qd:qd + kvd].reshape(1, hkv, hd)
    k_ref = O.rope_llama(k_new, pos, theta).to(torch.bfloat16).reshape(1, kvd)
    assert torch.equal(r_out.cpu(), res)
    assert_close_bf16(q_out, q_ref, what="rotated q")
    assert_close_bf16(kc[L - 1:L], k_ref, what="rotated k slot")
    assert_close_bf16(vc[L - 1:L], qkv[:, qd + kvd:], what="v slot")
    assert kc[L:].abs().sum() == 0 and vc[L:].abs().sum() == 0
    # attention over the rotated cache without RoPE == RoPE-on-read over un-rotated keys
    k_all = torch.cat([k_prev, k_new.to(torch.bfloat16)])
    v_all = torch.cat([v_prev, qkv[:, qd + kvd:].reshape(1, hkv, hd)])
    ref = O.attention_decode(qkv[:, :qd].reshape(1, hq, hd), k_all, v_all, L,
                             O.AttnCtx(hq, hkv, hd, rope_theta=theta, q_rope_pos_offset=pos_off,
                                       k_rope_pos_offset=pos_off))
    actx = C.make_attention_ctx(hq, hkv, hd, rope=False)
    ws = torch.zeros(C.load().efm_attention_decode_workspace_bytes(actx, rows), dtype=torch.uint8, device=gpu)
    o = torch.empty(1, hq, hd, dtype=torch.bfloat16, device=gpu)
    C.call("efm_attention_decode", actx, ptr(q_out), ptr(kc), ptr(vc), ptr(o), 0, ptr(d_len), rows, ptr(ws),
           ws.numel(), stream())
    torch.cuda.synchronize()
    assert_close_bf16(o, ref, what="attention over the rotated cache")


def test_decode_front_half_7b_16k_engine_chain(gpu):
    """The decode front half of one Qwen2.5-7B-shaped layer at C5's context, through the
    C-ABI chain the engine runs: norm + QKV with q and the new key rotated in the epilogue
    (slot 16447), decode attention over 16,448 rotated cache rows (28/4 heads: the 8-wave
    kernel, 58 splits of 288 keys of a 16,512-row cache, then the split merge kernel), and
    the o_proj GEMV; against the oracle's layer with RoPE on read over the un-rotated keys
    (Appendix-A rounding points)."""
    torch.manual_seed(21)
    hidden, hq, hkv, hd, eps, theta = 3584, 28, 4, 128, 1e-6, 1.0e6
    L, max_kv = 16448, 16512
    qd, kvd = hq * hd, hkv * hd
    h = torch.randn(1, hidden, dtype=torch.bfloat16)
    r = torch.randn(1, hidden, dtype=torch.bfloat16)
    nw = (1 + 0.1 * torch.randn(hidden)).to(torch.bfloat16)
    W = (torch.randn(qd + 2 * kvd, hidden) * 0.02).to(torch.bfloat16)
    b = (torch.randn(qd + 2 * kvd) * 0.02).to(torch.bfloat16)
    Wo = (torch.randn(hidden, qd) * 0.02).to(torch.bfloat16)
    k_prev = torch.randn(L - 1, hkv, hd, dtype=torch.bfloat16)
    v_prev = torch.randn(L - 1, hkv, hd, dtype=torch.bfloat16)
    kc = torch.full((max_kv, kvd), float("nan"), dtype=torch.bfloat16)
    vc = torch.full((max_kv, kvd), float("nan"), dtype=torch.bfloat16)
    kc[: L - 1] = O.rope_llama(k_prev, torch.arange(L - 1), theta).to(torch.bfloat16).reshape(L - 1, kvd)
    vc[: L - 1] = v_prev.reshape(L - 1, kvd)
    kc, vc = kc.to(gpu), vc.to(gpu)
    d_len = torch.tensor([L], dtype=torch.int32, device=gpu)
    hg, rg, nwg, Wg, bg, Wog = (t.to(gpu) for t in (h, r, nw, W, b, Wo))
    q = torch.empty(1, qd, dtype=torch.bfloat16, device=gpu)
    r_out = torch.empty(1, hidden, dtype=torch.bfloat16, device=gpu)
    attn = torch.empty(1, qd, dtype=torch.bfloat16, device=gpu)
    a = torch.empty(1, hidden, dtype=torch.bfloat16, device=gpu)
    cq = C.make_attention_ctx(hq, hkv, hd, rope_theta=theta)
    ca = C.make_attention_ctx(hq, hkv, hd, rope=False)
    ws = torch.zeros(C.load().efm_attention_decode_workspace_bytes(ca, max_kv), dtype=torch.uint8, device=gpu)
    C.call("efm_decode_norm_qkv_rope", cq, hidden, eps, ptr(hg), ptr(rg), ptr(r_out), ptr(nwg), ptr(Wg), ptr(bg),
           ptr(q), ptr(kc), ptr(vc), ptr(d_len), stream())
    C.call("efm_attention_decode", ca, ptr(q), ptr(kc), ptr(vc), ptr(attn), 0, ptr(d_len), max_kv, ptr(ws), ws.numel(),
           stream())
    C.call("efm_linear", 1, qd, hidden, ptr(attn), ptr(Wog), None, ptr(a), C.EFM_DTYPE_BF16, stream())
    torch.cuda.synchronize()
    n, res = O.fused_add_rms_norm(h, r, nw, eps)
    qkv = O.linear(n, W, b)
    k_all = torch.cat([k_prev, qkv[:, qd:qd + kvd].reshape(1, hkv, hd)])
    v_all = torch.cat([v_prev, qkv[:, qd + kvd:].reshape(1, hkv, hd)])
    o_ref = O.attention_decode(qkv[:, :qd].reshape(1, hq, hd), k_all, v_all, L,
                               O.AttnCtx(hq, hkv, hd, rope_theta=theta)).reshape(1, qd)
    a_ref = O.linear(o_ref, Wo)
    assert torch.equal(r_out.cpu(), res)
    assert torch.isfinite(attn.float()).all()
    assert_close_bf16(attn, o_ref, what="attention over 16,448 rows")
    assert_close_bf16(a, a_ref, what="o_proj of the attention output")
    assert torch.isnan(kc[L:].float()).all(), "rows past the newest must not be written"
    assert_close_bf16(vc[L - 1:L], qkv[:, qd + kvd:], what="v slot")


@pytest.mark.parametrize("hidden,inter", [(1536, 8960), (896, 4864), (3584, 18944)])
def test_decode_norm_gate_up_swiglu_matches_unfused(gpu, hidden, inter):
    torch.manual_seed(0)
    eps = 1e-6
    a = torch.randn(1, hidden, dtype=torch.bfloat16)
    r = torch.randn(1, hidden, dtype=torch.bfloat16)
    nw = (1 + 0.1 * torch.randn(hidden)).to(torch.bfloat16)
    W = (torch.randn(2 * inter, hidden) * 0.05).to(torch.bfloat16)
    out = torch.empty(1, inter, dtype=torch.bfloat16, device=gpu)
    r_out = torch.empty(1, hidden, dtype=torch.bfloat16, device=gpu)
    ag, rg, nwg, Wg = a.to(gpu), r.to(gpu), nw.to(gpu), W.to(gpu)
    C.call("efm_decode_norm_gate_up_swiglu", hidden, inter, eps, ptr(ag), ptr(rg), ptr(r_out), ptr(nwg), ptr(Wg),
           ptr(out), stream())
    torch.cuda.synchronize()
    n2, res = O.fused_add_rms_norm(a, r, nw, eps)
    assert torch.equal(r_out.cpu(), res)
    assert_close_bf16(out, O.gate_up_swiglu(n2, W), rtol=2e-2, atol=2e-2)


@pytest.mark.parametrize("hidden,vocab", [(1536, 151936), (896, 151936)])
def test_decode_norm_lm_head_top1_matches_unfused(gpu, hidden, vocab):
    torch.manual_seed(2)
    eps = 1e-6
    h = torch.randn(1, hidden, dtype=torch.bfloat16)
    r = torch.randn(1, hidden, dtype=torch.bfloat16)
    nw = (1 + 0.1 * torch.randn(hidden)).to(torch.bfloat16)
    W = (torch.randn(vocab, hidden) * 0.02).to(torch.bfloat16)
    ws = torch.zeros(C.load().efm_lm_head_top1_workspace_bytes(vocab), dtype=torch.uint8, device=gpu)
    tok = torch.full((1,), -1, dtype=torch.int32, device=gpu)
    hg, rg, nwg, Wg = h.to(gpu), r.to(gpu), nw.to(gpu), W.to(gpu)
    C.call("efm_decode_norm_lm_head_top1", hidden, vocab, eps, ptr(hg), ptr(rg), ptr(nwg), ptr(Wg), ptr(tok),
           ptr(ws), ws.numel(), stream())
    torch.cuda.synchronize()
    x, _ = O.fused_add_rms_norm(h, r, nw, eps)
    assert _top1_ref_ok(O.linear(x, W, out_f32=True)[0], int(tok.item()))


PREFILL_CASES = [
    pytest.param(12, 2, 128, 512, 512, id="1p5b_s512"),
    pytest.param(12, 2, 128, 37, 37, id="1p5b_s37"),
    pytest.param(14, 2, 64, 200, 200, id="0p5b_s200"),
    pytest.param(16, 2, 128, 300, 1100, id="3b_prefix800"),
    pytest.param(28, 4, 128, 1, 65, id="7b_s1_prefix64"),
    pytest.param(16, 2, 128, 1344, 1344, id="vl3b_s1344"),
]


@pytest.mark.parametrize("hq,hkv,hd,S,L", PREFILL_CASES)
def test_attention_prefill_matches_oracle(gpu, hq, hkv, hd, S, L):
    torch.manual_seed(0)
    q = torch.randn(S, hq, hd, dtype=torch.bfloat16)
    k = torch.randn(L, hkv, hd, dtype=torch.bfloat16)
    v = torch.randn(L, hkv, hd, dtype=torch.bfloat16)
    ref = O.attention_prefill(q, k, v, O.AttnCtx(hq, hkv, hd, q_rope_pos_offset=L - S), causal=True)
    ctx = C.make_attention_ctx(hq, hkv, hd, q_rope_pos_offset=L - S)
    qg, kg, vg = q.to(gpu), k.to(gpu), v.to(gpu)
    o = torch.empty(S, hq * hd, dtype=torch.bfloat16, device=gpu)
    C.call("efm_attention_prefill", ctx, ptr(qg), ptr(kg), ptr(vg), ptr(o), S, L, 1, stream())
    torch.cuda.synchronize()
    # P is rounded to bf16 before the PV product (as in FlashAttention-2 / FlashInfer)
    assert_close_bf16(o.reshape(S, hq, hd), ref, rtol=2e-2, atol=2e-2, what=f"prefill S={S} L={L}")


def test_attention_prefill_strided_qkv_no_rope_and_noncausal(gpu):
    """q taken from a fused QKV buffer (q_stride_n = qkv_total), pos NONE (M-RoPE models),
    and the non-causal mode."""
    torch.manual_seed(1)
    hq, hkv, hd, S = 16, 2, 128, 130
    tot = (hq + 2 * hkv) * hd
    qkv = torch.randn(S, tot, dtype=torch.bfloat16)
    q = qkv[:, : hq * hd].reshape(S, hq, hd)
    k = qkv[:, hq * hd: (hq + hkv) * hd].reshape(S, hkv, hd).contiguous()
    v = qkv[:, (hq + hkv) * hd:].reshape(S, hkv, hd).contiguous()
    for causal in (1, 0):
        ref = O.attention(q, k, v, torch.arange(S), O.AttnCtx(hq, hkv, hd, rope=False),
                          causal_offset=0 if causal else None)
        ctx = C.make_attention_ctx(hq, hkv, hd, rope=False, q_stride_n=tot, q_stride_h=hd)
        qkvg, kg, vg = qkv.to(gpu), k.to(gpu), v.to(gpu)
        o = torch.empty(S, hq * hd, dtype=torch.bfloat16, device=gpu)
        C.call("efm_attention_prefill", ctx, ptr(qkvg), ptr(kg), ptr(vg), ptr(o), S, S, causal, stream())
        torch.cuda.synchronize()
        assert_close_bf16(o.reshape(S, hq, hd), ref, rtol=2e-2, atol=2e-2, what=f"causal={causal}")


PIPE_CASES = [
    pytest.param(12, 2, 1, 1, 1, "none", id="s1"),
    pytest.param(12, 2, 77, 77, 1, "prerot", id="s77_prerot"),
    pytest.param(16, 2, 300, 1100, 1, "prerot", id="3b_prefix800_prerot"),
    pytest.param(28, 4, 513, 513, 0, "none", id="7b_s513_noncausal"),
    pytest.param(28, 4, 1000, 1000, 1, "none", id="7b_s1000"),
    pytest.param(16, 2, 1344, 1344, 1, "none", id="vl3b_s1344"),
    pytest.param(12, 2, 255, 1025, 0, "prerot", id="noncausal_prefix"),
    pytest.param(12, 2, 512, 512, 1, "none", id="1p5b_s512"),
]


@pytest.mark.parametrize("shape", ["2", "4", "8"])
@pytest.mark.parametrize("hq,hkv,S,L,causal,mode", PIPE_CASES)
def test_attention_prefill_pipelined_matches_oracle(gpu, knob, shape, hq, hkv, S, L, causal, mode):
    """head_dim 128 with keys already rotated (pos NONE, or RoPE on q only with
    k_already_prerotated) runs the global_load_lds ring kernel, in every workgroup shape
    (2 or 4 waves over a 2-deep ring, 8 waves over a 4-deep ring)."""
    knob(C.EFM_KNOB_PREFILL_SHAPE, int(shape))
    torch.manual_seed(S + L)
    hd = 128
    q = torch.randn(S, hq, hd, dtype=torch.bfloat16)
    k = torch.randn(L, hkv, hd, dtype=torch.bfloat16)
    v = torch.randn(L, hkv, hd, dtype=torch.bfloat16)
    if mode == "none":
        octx = O.AttnCtx(hq, hkv, hd, rope=False)
        ctx = C.make_attention_ctx(hq, hkv, hd, rope=False)
        kin = k
    else:
        octx = O.AttnCtx(hq, hkv, hd, q_rope_pos_offset=L - S)
        ctx = C.make_attention_ctx(hq, hkv, hd, q_rope_pos_offset=L - S, k_already_prerotated=True)
        kin = O.rope_llama(k, torch.arange(L), 1.0e6).to(torch.bfloat16)
    ref = O.attention(q, k, v, torch.arange(S) + (L - S), octx, causal_offset=(L - S) if causal else None)
    qg, kg, vg = q.to(gpu), kin.to(gpu), v.to(gpu)
    o = torch.empty(S, hq * hd, dtype=torch.bfloat16, device=gpu)
    C.call("efm_attention_prefill", ctx, ptr(qg), ptr(kg), ptr(vg), ptr(o), S, L, causal, stream())
    torch.cuda.synchronize()
    assert_close_bf16(o.reshape(S, hq, hd), ref, rtol=2e-2, atol=2e-2, what=f"pipelined S={S} L={L} {mode}")


@pytest.mark.parametrize("shape", ["2", "4", "8"])
def test_attention_prefill_pipelined_matches_register_kernel_c4(gpu, knob, shape):
    """BASELINE C4 shape (28/4 heads, S = 4096, causal): the pipelined kernel (every
    workgroup shape) against the register-staged one (EFM_KNOB_PREFILL_REGISTER)."""
    knob(C.EFM_KNOB_PREFILL_SHAPE, int(shape))
    torch.manual_seed(44)
    hq, hkv, hd, S = 28, 4, 128, 4096
    q = torch.randn(S, hq, hd, dtype=torch.bfloat16, device=gpu)
    k = torch.randn(S, hkv, hd, dtype=torch.bfloat16, device=gpu)
    v = torch.randn(S, hkv, hd, dtype=torch.bfloat16, device=gpu)
    ctx = C.make_attention_ctx(hq, hkv, hd, rope=False)
    outs = []
    for pipe in ("1", "0"):
        knob(C.EFM_KNOB_PREFILL_REGISTER, 1 if pipe == "0" else 0)
        o = torch.empty(S, hq * hd, dtype=torch.bfloat16, device=gpu)
        C.call("efm_attention_prefill", ctx, ptr(q), ptr(k), ptr(v), ptr(o), S, S, 1, stream())
        torch.cuda.synchronize()
        outs.append(o)
    assert torch.isfinite(outs[0].float()).all()
    assert_close_bf16(outs[0], outs[1], rtol=2e-2, atol=2e-2, what="pipelined vs register kernel")
    # spot rows against the oracle (first, middle, last query rows of every head)
    for r in (0, 1, 2047, 4095):
        ref = O.attention(q[r:r + 1].cpu(), k[:r + 1].cpu(), v[:r + 1].cpu(), torch.tensor([r]),
                          O.AttnCtx(hq, hkv, hd, rope=False), causal_offset=None)
        assert_close_bf16(outs[0][r].reshape(1, hq, hd), ref, rtol=2e-2, atol=2e-2, what=f"C4 row {r} vs oracle")


def test_attention_prefill_last_row_equals_decode(gpu):
    """The last prefill row equals single-query decode over the same cache (the
    reference's prefill/decode consistency)."""
    torch.manual_seed(2)
    hq, hkv, hd, L = 12, 2, 128, 700
    q = torch.randn(L, hq, hd, dtype=torch.bfloat16, device=gpu)
    k = torch.randn(L, hkv, hd, dtype=torch.bfloat16, device=gpu)
    v = torch.randn(L, hkv, hd, dtype=torch.bfloat16, device=gpu)
    o = torch.empty(L, hq * hd, dtype=torch.bfloat16, device=gpu)
    C.call("efm_attention_prefill", C.make_attention_ctx(hq, hkv, hd), ptr(q), ptr(k), ptr(v), ptr(o), L, L, 1,
           stream())
    dec, _ = _decode(C.make_attention_ctx(hq, hkv, hd), q[-1:].contiguous(), k, v, L)
    assert_close_bf16(o[-1].reshape(1, hq, hd), dec, rtol=2e-2, atol=2e-2)


def test_mrope_matches_oracle(gpu):
    torch.manual_seed(0)
    S, hq, hkv, hd = 70, 16, 2, 128
    sections = (16, 24, 24)
    q = torch.randn(S, hq, hd, dtype=torch.bfloat16)
    k = torch.randn(S, hkv, hd, dtype=torch.bfloat16)
    pos = torch.stack([torch.zeros(S, dtype=torch.int32), torch.arange(S, dtype=torch.int32) // 7,
                       torch.arange(S, dtype=torch.int32) % 7]) + 3
    qg, kg, pg = q.to(gpu), k.to(gpu), pos.to(gpu)
    C.call("efm_mrope", ptr(qg), ptr(kg), ptr(pg), S, S, hq, hkv, hd, 0, 0, *sections, 1.0e6, 1.0, stream())
    torch.cuda.synchronize()
    assert_close_bf16(qg, O.mrope(q, pos, sections, 1.0e6), what="mrope q")
    assert_close_bf16(kg, O.mrope(k, pos, sections, 1.0e6), what="mrope k")


def test_decode_mrope_write_kv(gpu):
    torch.manual_seed(0)
    hq, hkv, hd = 16, 2, 128
    sections = (16, 24, 24)
    qkv = torch.randn(1, (hq + 2 * hkv) * hd, dtype=torch.bfloat16)
    pos = torch.tensor([40, 41, 45], dtype=torch.int32)
    rows = 50
    qkvg, pg = qkv.to(gpu), pos.to(gpu)
    kc = torch.zeros(rows, hkv * hd, dtype=torch.bfloat16, device=gpu)
    vc = torch.zeros(rows, hkv * hd, dtype=torch.bfloat16, device=gpu)
    qd = torch.empty(1, hq * hd, dtype=torch.bfloat16, device=gpu)
    d_len = torch.tensor([31], dtype=torch.int32, device=gpu)
    base = qkvg.data_ptr()
    C.call("efm_decode_mrope_write_kv", base, base + hq * hd * 2, base + (hq + hkv) * hd * 2, ptr(qd), ptr(kc),
           ptr(vc), hq, hkv, hd, ptr(pg), *sections, 1.0e6, 1.0, ptr(d_len), stream())
    torch.cuda.synchronize()
    q = qkv[:, : hq * hd].reshape(1, hq, hd)
    k = qkv[:, hq * hd: (hq + hkv) * hd].reshape(1, hkv, hd)
    p3 = pos.reshape(3, 1)
    assert_close_bf16(qd.reshape(1, hq, hd), O.mrope(q, p3, sections, 1.0e6))
    assert_close_bf16(kc[30].reshape(1, hkv, hd), O.mrope(k, p3, sections, 1.0e6))
    assert torch.equal(vc[30].cpu(), qkv[0, (hq + hkv) * hd:])
    assert kc[:30].abs().sum() == 0 and kc[31:].abs().sum() == 0


def test_finalize_indexed(gpu):
    resp = torch.full((8,), -1, dtype=torch.int32, device=gpu)
    step = torch.zeros(1, dtype=torch.int32, device=gpu)
    d_len = torch.tensor([10], dtype=torch.int32, device=gpu)
    tok = torch.zeros(1, dtype=torch.int32, device=gpu)
    for i in range(10):
        tok.fill_(100 + i)
        C.call("efm_finalize_decode_token_indexed", ptr(tok), ptr(resp), ptr(step), ptr(d_len), 8, stream())
    torch.cuda.synchronize()
    assert resp.cpu().tolist() == [100 + i for i in range(8)]
    assert int(step.item()) == 10 and int(d_len.item()) == 20


@pytest.mark.parametrize("hq,hkv,hd,hidden", [pytest.param(12, 2, 128, 1536, id="1p5b"),
                                               pytest.param(14, 2, 64, 896, id="0p5b"),
                                               pytest.param(16, 2, 128, 2048, id="vl3b")])
@pytest.mark.parametrize("max_kv,kv_len,rope", [(768, 1, True), (768, 100, True), (768, 640, True),
                                                (768, 767, True), (768, 640, False), (1024, 1024, False),
                                                (1024, 129, True)])
def test_decode_attention_partials_merge_o_proj(gpu, hq, hkv, hd, hidden, max_kv, kv_len, rope):
    """Split partials + merge folded into the o_proj GEMV == attention then o_proj, on
    rotate-on-read and rotated caches, up to the 1024 rows (8 splits) it takes."""
    torch.manual_seed(0)
    q = torch.randn(1, hq, hd, dtype=torch.bfloat16)
    k = torch.randn(max_kv, hkv, hd, dtype=torch.bfloat16)
    v = torch.randn(max_kv, hkv, hd, dtype=torch.bfloat16)
    wo = (torch.randn(hidden, hq * hd) * 0.02).to(torch.bfloat16)
    ctx = C.make_attention_ctx(hq, hkv, hd, rope=rope)
    qg, kg, vg, wg = q.to(gpu), k.to(gpu), v.to(gpu), wo.to(gpu)
    d_len = torch.tensor([kv_len], dtype=torch.int32, device=gpu)
    ws = torch.zeros(C.load().efm_attention_decode_workspace_bytes(ctx, max_kv), dtype=torch.uint8, device=gpu)
    out = torch.empty(1, hidden, dtype=torch.bfloat16, device=gpu)
    for _ in range(2):
        C.call("efm_decode_attention_partials", ctx, ptr(qg), ptr(kg), ptr(vg), ptr(d_len), max_kv, ptr(ws),
               ws.numel(), stream())
        C.call("efm_decode_attention_merge_o_proj", ctx, ptr(d_len), max_kv, ptr(ws), ws.numel(), ptr(wg), hidden,
               ptr(out), stream())
    torch.cuda.synchronize()
    att = O.attention_decode(q, k, v, kv_len, O.AttnCtx(hq, hkv, hd, rope=rope))
    ref = O.linear(att.reshape(1, hq * hd), wo)
    assert_close_bf16(out, ref, rtol=2e-2, atol=2e-2, what=f"partials+merge max={max_kv} kv={kv_len}")


@pytest.mark.parametrize("hq,hkv,hidden", [pytest.param(14, 2, 896, id="0p5b"), pytest.param(16, 2, 1024, id="w1024"),
                                            pytest.param(8, 8, 512, id="mha")])
@pytest.mark.parametrize("max_kv,kv_len", [(1, 1), (40, 17), (1025, 1025), (1025, 1), (1025, 64), (1025, 65),
                                           (1536, 1536), (1536, 700)])
def test_decode_attention_partials_merge_o_proj_narrow(gpu, hq, hkv, hidden, max_kv, kv_len):
    """head_dim 64 with query widths up to 1024: one-wave partials of 32 / 64 keys (up to
    24 splits, caches up to 1536 rows) merged in the narrow o_proj prologue == the oracle's
    attention then o_proj, and == efm_attention_decode + efm_linear to rounding. Rows past
    the length hold Inf / NaN and must not leak in; two calls in a row agree bit for bit."""
    hd = 64
    torch.manual_seed(1)
    q = torch.randn(1, hq, hd, dtype=torch.bfloat16)
    k = torch.randn(max_kv, hkv, hd, dtype=torch.bfloat16)
    v = torch.randn(max_kv, hkv, hd, dtype=torch.bfloat16)
    wo = (torch.randn(hidden, hq * hd) * 0.02).to(torch.bfloat16)
    ctx = C.make_attention_ctx(hq, hkv, hd, rope=False)
    lib = C.load()
    assert lib.efm_decode_attention_merge_o_proj_supported(ctx, max_kv) == C.EFM_OK
    qg, kg, vg, wg = q.to(gpu), k.to(gpu), v.to(gpu), wo.to(gpu)
    kg[kv_len:] = float("inf")
    vg[kv_len:] = float("nan")
    d_len = torch.tensor([kv_len], dtype=torch.int32, device=gpu)
    ws = torch.zeros(lib.efm_attention_decode_workspace_bytes(ctx, max_kv), dtype=torch.uint8, device=gpu)
    outs = []
    for _ in range(2):
        out = torch.empty(1, hidden, dtype=torch.bfloat16, device=gpu)
        C.call("efm_decode_attention_partials", ctx, ptr(qg), ptr(kg), ptr(vg), ptr(d_len), max_kv, ptr(ws),
               ws.numel(), stream())
        C.call("efm_decode_attention_merge_o_proj", ctx, ptr(d_len), max_kv, ptr(ws), ws.numel(), ptr(wg), hidden,
               ptr(out), stream())
        outs.append(out)
    att = torch.empty(1, hq * hd, dtype=torch.bfloat16, device=gpu)
    ref_gpu = torch.empty(1, hidden, dtype=torch.bfloat16, device=gpu)
    C.call("efm_attention_decode", ctx, ptr(qg), ptr(kg), ptr(vg), ptr(att), 0, ptr(d_len), max_kv, ptr(ws),
           ws.numel(), stream())
    C.call("efm_linear", 1, hq * hd, hidden, ptr(att), ptr(wg), None, ptr(ref_gpu), C.EFM_DTYPE_BF16, stream())
    torch.cuda.synchronize()
    assert torch.equal(outs[0], outs[1])
    assert torch.isfinite(outs[0].float()).all()
    ref = O.linear(O.attention_decode(q, k[:kv_len], v[:kv_len], kv_len, O.AttnCtx(hq, hkv, hd, rope=False))
                   .reshape(1, hq * hd), wo)
    what = f"narrow partials+merge {hq}/{hkv} max={max_kv} kv={kv_len}"
    assert_close_bf16(outs[0], ref, rtol=2e-2, atol=2e-2, what=what)
    assert_close_bf16(outs[0], ref_gpu, rtol=2e-2, atol=2e-2, what=what + " vs attention_decode + linear")


@pytest.mark.parametrize("hq,hkv,hidden", [pytest.param(12, 2, 1536, id="1p5b"), pytest.param(16, 2, 2048, id="vl3b"),
                                            pytest.param(16, 4, 2048, id="g4")])
@pytest.mark.parametrize("max_kv,kv_len", [(96, 96), (256, 1), (384, 200), (1025, 1025), (1280, 700), (1536, 1536),
                                           (1536, 1)])
def test_decode_attention_partials_merge_o_proj_head_dim_128_plans(gpu, hq, hkv, hidden, max_kv, kv_len):
    """head_dim 128 beyond the 8-split merge: one-tile (32-key) partials up to 12 splits at
    short caches, and 9-12 splits of 128 keys (the 12-slot prologue) at 1025-1536 rows, ==
    the oracle's attention then o_proj, and == efm_attention_decode + efm_linear to rounding.
    Rows past the length hold Inf / NaN; two calls in a row agree bit for bit."""
    hd = 128
    torch.manual_seed(4)
    q = torch.randn(1, hq, hd, dtype=torch.bfloat16)
    k = torch.randn(max_kv, hkv, hd, dtype=torch.bfloat16)
    v = torch.randn(max_kv, hkv, hd, dtype=torch.bfloat16)
    wo = (torch.randn(hidden, hq * hd) * 0.02).to(torch.bfloat16)
    ctx = C.make_attention_ctx(hq, hkv, hd, rope=False)
    lib = C.load()
    assert lib.efm_decode_attention_merge_o_proj_supported(ctx, max_kv) == C.EFM_OK
    qg, kg, vg, wg = q.to(gpu), k.to(gpu), v.to(gpu), wo.to(gpu)
    kg[kv_len:] = float("inf")
    vg[kv_len:] = float("nan")
    d_len = torch.tensor([kv_len], dtype=torch.int32, device=gpu)
    ws = torch.zeros(lib.efm_attention_decode_workspace_bytes(ctx, max_kv), dtype=torch.uint8, device=gpu)
    outs = []
    for _ in range(2):
        out = torch.empty(1, hidden, dtype=torch.bfloat16, device=gpu)
        C.call("efm_decode_attention_partials", ctx, ptr(qg), ptr(kg), ptr(vg), ptr(d_len), max_kv, ptr(ws),
               ws.numel(), stream())
        C.call("efm_decode_attention_merge_o_proj", ctx, ptr(d_len), max_kv, ptr(ws), ws.numel(), ptr(wg), hidden,
               ptr(out), stream())
        outs.append(out)
    att = torch.empty(1, hq * hd, dtype=torch.bfloat16, device=gpu)
    ref_gpu = torch.empty(1, hidden, dtype=torch.bfloat16, device=gpu)
    C.call("efm_attention_decode", ctx, ptr(qg), ptr(kg), ptr(vg), ptr(att), 0, ptr(d_len), max_kv, ptr(ws),
           ws.numel(), stream())
    C.call("efm_linear", 1, hq * hd, hidden, ptr(att), ptr(wg), None, ptr(ref_gpu), C.EFM_DTYPE_BF16, stream())
    torch.cuda.synchronize()
    assert torch.equal(outs[0], outs[1])
    assert torch.isfinite(outs[0].float()).all()
    ref = O.linear(O.attention_decode(q, k[:kv_len], v[:kv_len], kv_len, O.AttnCtx(hq, hkv, hd, rope=False))
                   .reshape(1, hq * hd), wo)
    what = f"head_dim 128 partials+merge {hq}/{hkv} max={max_kv} kv={kv_len}"
    assert_close_bf16(outs[0], ref, rtol=2e-2, atol=2e-2, what=what)
    assert_close_bf16(outs[0], ref_gpu, rtol=2e-2, atol=2e-2, what=what + " vs attention_decode + linear")


def _sage_inputs(S, L, hq, hkv, hd, seed=0, gpu=None):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(S, hq, hd, generator=g).to(torch.bfloat16)
    k = (torch.randn(L, hkv, hd, generator=g) + 0.5).to(torch.bfloat16)  # non-zero channel means
    v = torch.randn(L, hkv, hd, generator=g).to(torch.bfloat16)
    return q, k, v


@pytest.mark.parametrize("S,L,hq,hkv,hd", [(300, 300, 28, 4, 128), (129, 257, 4, 2, 64), (1, 40, 8, 1, 128)])
def test_sage_quantize_bit_exact(gpu, S, L, hq, hkv, hd):
    """The int8 path is exact: Q8 / K8 / scales equal the oracle bit for bit (K8 and its
    scales recomputed from the GPU's float64-accumulated K mean)."""
    q, k, v = _sage_inputs(S, L, hq, hkv, hd)
    ctx = C.make_attention_ctx(hq, hkv, hd, rope=False)
    qg, kg = q.to(gpu), k.to(gpu)
    nbq, nbk = (S + 127) // 128, (L + 127) // 128
    q8 = torch.empty(S, hq, hd, dtype=torch.int8, device=gpu)
    k8 = torch.empty(L, hkv, hd, dtype=torch.int8, device=gpu)
    sq = torch.empty(nbq, hq, dtype=torch.float32, device=gpu)
    sk = torch.empty(nbk, hkv, dtype=torch.float32, device=gpu)
    km = torch.empty(hkv, hd, dtype=torch.float32, device=gpu)
    C.call("efm_sage_quantize", ctx, ptr(qg), ptr(kg), S, L, ptr(q8), ptr(sq), ptr(k8), ptr(sk), ptr(km), stream())
    torch.cuda.synchronize()
    ref_km = O.sage_kmean(k)
    torch.testing.assert_close(km.cpu(), ref_km, rtol=2e-7, atol=1e-7)
    rq8, rsq = O.sage_quant_blocks(q.float())
    rk8, rsk = O.sage_quant_blocks(k.float() - km.cpu()[None])
    assert torch.equal(q8.cpu(), rq8) and torch.equal(sq.cpu(), rsq)
    assert torch.equal(k8.cpu(), rk8) and torch.equal(sk.cpu(), rsk)


@pytest.mark.parametrize("S,L,hq,hkv,hd", [(300, 300, 28, 4, 128), (129, 257, 4, 2, 64), (1, 40, 8, 1, 128),
                                           (4096, 4096, 28, 4, 128), (700, 1003, 8, 2, 128)])
def test_sage_attention_quantisation_equals_quantize_entry(gpu, S, L, hq, hkv, hd):
    """The attention entry point takes its K mean from float64 row-slice sums added up by
    the quantisation kernel; its K8 / K scales / K mean (left in the workspace) must equal
    efm_sage_quantize's (one workgroup per channel group) bit for bit."""
    q, k, v = _sage_inputs(S, L, hq, hkv, hd, seed=3)
    ctx = C.make_attention_ctx(hq, hkv, hd, rope=False)
    qg, kg, vg = q.to(gpu), k.to(gpu), v.to(gpu)
    nbq, nbk = (S + 127) // 128, (L + 127) // 128
    q8 = torch.empty(S, hq, hd, dtype=torch.int8, device=gpu)
    k8 = torch.empty(L, hkv, hd, dtype=torch.int8, device=gpu)
    sq = torch.empty(nbq, hq, dtype=torch.float32, device=gpu)
    sk = torch.empty(nbk, hkv, dtype=torch.float32, device=gpu)
    km = torch.empty(hkv, hd, dtype=torch.float32, device=gpu)
    C.call("efm_sage_quantize", ctx, ptr(qg), ptr(kg), S, L, ptr(q8), ptr(sq), ptr(k8), ptr(sk), ptr(km), stream())
    ws = torch.zeros(C.load().efm_attention_prefill_sage_int8_workspace_bytes(ctx, S, L), dtype=torch.uint8,
                     device=gpu)
    o = torch.empty(S, hq * hd, dtype=torch.bfloat16, device=gpu)
    C.call("efm_attention_prefill_sage_int8", ctx, ptr(qg), ptr(kg), ptr(vg), ptr(o), S, L, 1, ptr(ws), ws.numel(),
           stream())
    torch.cuda.synchronize()
    al = lambda x: (x + 255) // 256 * 256
    off_k8 = al(S * hq * hd)
    off_sk = off_k8 + al(L * hkv * hd) + al(nbq * hq * 4)
    off_km = off_sk + al(nbk * hkv * 4)
    w = ws.cpu()
    assert torch.equal(w[off_k8:off_k8 + L * hkv * hd].view(torch.int8).reshape(L, hkv, hd), k8.cpu())
    assert torch.equal(w[off_sk:off_sk + nbk * hkv * 4].view(torch.float32).reshape(nbk, hkv), sk.cpu())
    assert torch.equal(w[off_km:off_km + hkv * hd * 4].view(torch.float32).reshape(hkv, hd), km.cpu())
    torch.testing.assert_close(km.cpu(), O.sage_kmean(k), rtol=2e-7, atol=1e-7)


@pytest.mark.parametrize("S,L,hq,hkv,hd", [(512, 512, 28, 4, 128), (300, 700, 8, 2, 128), (200, 200, 14, 2, 64)])
def test_sage_attention_matches_oracle(gpu, S, L, hq, hkv, hd):
    q, k, v = _sage_inputs(S, L, hq, hkv, hd, seed=1)
    ctx = C.make_attention_ctx(hq, hkv, hd, rope=False)
    qg, kg, vg = q.to(gpu), k.to(gpu), v.to(gpu)
    o = torch.empty(S, hq * hd, dtype=torch.bfloat16, device=gpu)
    ws = torch.zeros(C.load().efm_attention_prefill_sage_int8_workspace_bytes(ctx, S, L), dtype=torch.uint8,
                     device=gpu)
    C.call("efm_attention_prefill_sage_int8", ctx, ptr(qg), ptr(kg), ptr(vg), ptr(o), S, L, 1, ptr(ws), ws.numel(),
           stream())
    torch.cuda.synchronize()
    ref = O.sage_attention(q, k, v, hkv, causal=True)
    assert_close_bf16(o.reshape(S, hq, hd), ref, rtol=2e-2, atol=2e-2, what="sage vs int8 oracle")
    bf = O.attention_prefill(q, k, v, O.AttnCtx(hq, hkv, hd, rope=False), causal=True)
    err = (o.reshape(S, hq, hd).float().cpu() - bf.float()).abs()
    assert float(err.mean()) < 5e-3 and float(err.max()) < 0.1, (float(err.mean()), float(err.max()))


def test_sage_attention_c4_shape_vs_bf16_kernel(gpu):
    """BASELINE config 4 at full size (28/4 heads, hd 128, S 4096, causal): int8 path vs
    the bf16 MFMA prefill kernel on the same inputs (size-independent error bounds)."""
    S, hq, hkv, hd = 4096, 28, 4, 128
    g = torch.Generator(device=gpu).manual_seed(7)
    q = torch.randn(S, hq, hd, generator=g, device=gpu).to(torch.bfloat16)
    k = torch.randn(S, hkv, hd, generator=g, device=gpu).to(torch.bfloat16)
    v = torch.randn(S, hkv, hd, generator=g, device=gpu).to(torch.bfloat16)
    ctx = C.make_attention_ctx(hq, hkv, hd, rope=False)
    o8 = torch.empty(S, hq * hd, dtype=torch.bfloat16, device=gpu)
    ob = torch.empty(S, hq * hd, dtype=torch.bfloat16, device=gpu)
    ws = torch.zeros(C.load().efm_attention_prefill_sage_int8_workspace_bytes(ctx, S, S), dtype=torch.uint8,
                     device=gpu)
    C.call("efm_attention_prefill_sage_int8", ctx, ptr(q), ptr(k), ptr(v), ptr(o8), S, S, 1, ptr(ws), ws.numel(),
           stream())
    C.call("efm_attention_prefill", ctx, ptr(q), ptr(k), ptr(v), ptr(ob), S, S, 1, stream())
    torch.cuda.synchronize()
    err = (o8.float() - ob.float()).abs()
    cos = torch.nn.functional.cosine_similarity(o8.float().flatten(), ob.float().flatten(), dim=0)
    assert float(err.mean()) < 5e-3 and float(cos) > 0.999, (float(err.mean()), float(cos))


@pytest.mark.parametrize("shape", ["4", "8"])
@pytest.mark.parametrize("S,L,causal", [(4096, 4096, 1), (1000, 1300, 1), (77, 77, 0)])
def test_sage_attention_pipelined_matches_register_kernel(gpu, knob, shape, S, L, causal):
    """head_dim 128 runs the global_load_lds ring kernel (both workgroup shapes); it must
    agree with the register-staged kernel (EFM_KNOB_PREFILL_REGISTER) on the same inputs."""
    knob(C.EFM_KNOB_PREFILL_SHAPE, int(shape))
    hq, hkv, hd = 28, 4, 128
    g = torch.Generator(device=gpu).manual_seed(S + L)
    q = torch.randn(S, hq, hd, generator=g, device=gpu).to(torch.bfloat16)
    k = torch.randn(L, hkv, hd, generator=g, device=gpu).to(torch.bfloat16)
    v = torch.randn(L, hkv, hd, generator=g, device=gpu).to(torch.bfloat16)
    ctx = C.make_attention_ctx(hq, hkv, hd, rope=False)
    ws = torch.zeros(C.load().efm_attention_prefill_sage_int8_workspace_bytes(ctx, S, L), dtype=torch.uint8,
                     device=gpu)
    outs = []
    for pipe in ("1", "0"):
        knob(C.EFM_KNOB_PREFILL_REGISTER, 1 if pipe == "0" else 0)
        o = torch.empty(S, hq * hd, dtype=torch.bfloat16, device=gpu)
        C.call("efm_attention_prefill_sage_int8", ctx, ptr(q), ptr(k), ptr(v), ptr(o), S, L, causal, ptr(ws),
               ws.numel(), stream())
        torch.cuda.synchronize()
        outs.append(o)
    assert torch.isfinite(outs[0].float()).all()
    assert_close_bf16(outs[0], outs[1], rtol=2e-2, atol=2e-2, what="sage pipelined vs register kernel")


@pytest.mark.parametrize("hq,hkv", [(12, 2), (28, 4), (16, 2), (8, 8)])
@pytest.mark.parametrize("kv_len,max_kv", [(1, 1), (100, 128), (767, 768), (1025, 2000), (16385, 16513)])
def test_decode_attention_lds_kernel_matches_register_kernel(gpu, knob, hq, hkv, kv_len, max_kv):
    """head_dim 128 with a rotated cache runs the LDS-staged kernel; it must agree with
    the register kernel (EFM_KNOB_DECODE_REGISTER) on the same cache, through both the merged
    entry point and the partials + fused o_proj merge, and store the same rotated newest
    row. Rows past the length hold NaN."""
    _lds_vs_register(gpu, knob, hq, hkv, kv_len, max_kv)


@pytest.mark.parametrize("hq,hkv,kv_len,max_kv", [
    pytest.param(64, 64, 1057, 1100, id="288keys-partial-last-split"),
    pytest.param(64, 64, 1, 1100, id="288keys-one-row"),
    pytest.param(128, 64, 900, 1100, id="288keys-g2"),
    pytest.param(448, 64, 1100, 1100, id="288keys-g7-full"),
    pytest.param(256, 256, 257, 300, id="256keys-8-tiles"),
    pytest.param(28, 4, 16448, 16512, id="c5-58-splits"),
    pytest.param(28, 4, 16390, 16512, id="c5-short-last-split"),
    pytest.param(28, 4, 18432, 18432, id="c5-64-splits-9-tiles"),
])
def test_decode_attention_wide_kernel_matches_register_kernel(gpu, knob, hq, hkv, kv_len, max_kv):
    """Plans past 512 splits of 128 keys run the 8-wave kernel (one workgroup per CU, splits
    of 256-288 keys, every tile in LDS; wave 0 takes a ninth tile): same checks as the 4-wave kernel, including a split whose last tiles lie past the
    length and waves without a tile."""
    _lds_vs_register(gpu, knob, hq, hkv, kv_len, max_kv)


@pytest.mark.parametrize("hq,hkv,kv_len,max_kv,k_off", [
    pytest.param(64, 64, 1057, 1100, 0, id="288keys-partial-last-split"),
    pytest.param(64, 64, 1, 1100, 0, id="288keys-one-row"),
    pytest.param(128, 64, 900, 1100, 3, id="288keys-g2-koff"),
    pytest.param(448, 64, 1100, 1100, 0, id="288keys-g7-full"),
    pytest.param(256, 256, 257, 300, 0, id="256keys-8-tiles"),
    pytest.param(28, 4, 16448, 16512, 0, id="c5-7b-16k"),
    pytest.param(28, 4, 18400, 18432, 5, id="288keys-9-tiles-koff"),
])
def test_decode_attention_wide_kernel_rotate_on_read(gpu, knob, hq, hkv, kv_len, max_kv, k_off):
    """The reference's un-rotated cache (k_already_prerotated 0: every key rotated on read
    at j + k_rope_pos_offset, qwen2_5.cpp:602,624-638 and attention.cu:135-139) on plans
    that take the 8-wave kernel: against the oracle and the register-staged kernel, rows
    past the length NaN, and the cache left as it was (nothing is stored back)."""
    torch.manual_seed(kv_len + hq + 7)
    hd = 128
    q = torch.randn(1, hq, hd, dtype=torch.bfloat16)
    k0 = torch.randn(max_kv, hkv, hd, dtype=torch.bfloat16)
    v0 = torch.randn(max_kv, hkv, hd, dtype=torch.bfloat16)
    ref = O.attention_decode(q, k0, v0, kv_len, O.AttnCtx(hq, hkv, hd, k_rope_pos_offset=k_off))
    k0[kv_len:] = float("nan")
    v0[kv_len:] = float("nan")
    ctx = C.make_attention_ctx(hq, hkv, hd, k_rope_pos_offset=k_off)
    assert ctx.k_already_prerotated == 0
    qg, vg = q.reshape(1, hq * hd).to(gpu), v0.to(gpu)
    d_len = torch.tensor([kv_len], dtype=torch.int32, device=gpu)
    ws = torch.zeros(C.load().efm_attention_decode_workspace_bytes(ctx, max_kv), dtype=torch.uint8, device=gpu)
    outs = []
    for reg in (0, 1):
        knob(C.EFM_KNOB_DECODE_REGISTER, reg)
        k = k0.to(gpu)
        o = torch.empty_like(qg)
        C.call("efm_attention_decode", ctx, ptr(qg), ptr(k), ptr(vg), ptr(o), 0, ptr(d_len), max_kv, ptr(ws),
               ws.numel(), stream())
        torch.cuda.synchronize()
        outs.append(o)
        assert torch.equal(k[:kv_len].cpu(), k0[:kv_len]), "rotate-on-read must not store keys"
    assert torch.isfinite(outs[0].float()).all()
    assert_close_bf16(outs[0].reshape(1, hq, hd), ref, what=f"wide rotate-on-read L={kv_len}")
    assert_close_bf16(outs[0], outs[1], what="wide rotate-on-read vs register kernel")


def _lds_vs_register(gpu, knob, hq, hkv, kv_len, max_kv):
    torch.manual_seed(kv_len + hq)
    hd = 128
    q = torch.randn(1, hq * hd, dtype=torch.bfloat16, device=gpu)
    k0 = torch.randn(max_kv, hkv, hd, dtype=torch.bfloat16, device=gpu)
    v = torch.randn(max_kv, hkv, hd, dtype=torch.bfloat16, device=gpu)
    k0[kv_len:] = float("nan")
    v[kv_len:] = float("nan")
    ctx = C.make_attention_ctx(hq, hkv, hd)
    ctx.k_already_prerotated = C.EFM_K_PREROTATED_EXCEPT_NEWEST
    d_len = torch.tensor([kv_len], dtype=torch.int32, device=gpu)
    ws = torch.zeros(C.load().efm_attention_decode_workspace_bytes(ctx, max_kv), dtype=torch.uint8, device=gpu)
    outs, caches = [], []
    for lds in ("1", "0"):
        knob(C.EFM_KNOB_DECODE_REGISTER, 1 if lds == "0" else 0)
        k = k0.clone()
        o = torch.empty_like(q)
        C.call("efm_attention_decode", ctx, ptr(q), ptr(k), ptr(v), ptr(o), 0, ptr(d_len), max_kv, ptr(ws),
               ws.numel(), stream())
        torch.cuda.synchronize()
        outs.append(o)
        caches.append(k)
    assert torch.isfinite(outs[0].float()).all()
    assert_close_bf16(outs[0], outs[1], what="lds vs register decode kernel")
    assert torch.equal(caches[0][: kv_len - 1], k0[: kv_len - 1])
    # the newest row: both rotate with the same cos/sin table and rounding
    assert torch.equal(caches[0][kv_len - 1], caches[1][kv_len - 1])


@pytest.mark.parametrize("lds", ["0", "1"])
@pytest.mark.parametrize("kv_len,max_kv", [(161, 40000), (321, 70000), (1025, 40000), (129, 40000)])
def test_decode_newest_row_owned_by_one_split(gpu, knob, lds, kv_len, max_kv):
    """With keys-per-split not a multiple of 128 (large max_kv_len) a split's last round has
    idle tiles that lie in the next split; they must not touch the newest row, which only
    its owning split rotates and stores (regression: the idle tile stored zeros)."""
    knob(C.EFM_KNOB_DECODE_REGISTER, 1 if lds == "0" else 0)
    torch.manual_seed(0)
    hq, hkv, hd = 12, 2, 128
    q = torch.randn(1, hq * hd, dtype=torch.bfloat16, device=gpu)
    k = torch.randn(max_kv, hkv, hd, dtype=torch.bfloat16, device=gpu)
    v = torch.randn(max_kv, hkv, hd, dtype=torch.bfloat16, device=gpu)
    raw = k[kv_len - 1].clone().cpu()
    ctx = C.make_attention_ctx(hq, hkv, hd)
    ctx.k_already_prerotated = C.EFM_K_PREROTATED_EXCEPT_NEWEST
    d_len = torch.tensor([kv_len], dtype=torch.int32, device=gpu)
    ws = torch.zeros(C.load().efm_attention_decode_workspace_bytes(ctx, max_kv), dtype=torch.uint8, device=gpu)
    C.call("efm_decode_attention_partials", ctx, ptr(q), ptr(k), ptr(v), ptr(d_len), max_kv, ptr(ws), ws.numel(),
           stream())
    torch.cuda.synchronize()
    want = O.rope_llama(raw.unsqueeze(0), torch.tensor([kv_len - 1]), 1.0e6).to(torch.bfloat16)[0]
    assert_close_bf16(k[kv_len - 1], want, rtol=1e-2, atol=1e-2, what="newest row")
