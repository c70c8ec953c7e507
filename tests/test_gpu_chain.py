"""GPU tests of the persistent post-attention decode chain (efm_decode_layer_chain).

The chain must equal, bit for bit, the unfused sequence it replaces:
efm_decode_attention_merge_o_proj -> efm_decode_norm_gate_up_swiglu -> efm_linear (down)
-> efm_decode_norm_qkv of the next layer, whose kernels are themselves pinned to the
oracle in test_gpu_ops.py. It is also checked against the oracle directly, run several
times in a row (each launch advances the exchange tag), and on the last layer."""
import pytest
import torch

import efm_capi as C
from oracle import efm_oracle as O
from _util import assert_close_bf16, ptr, stream

pytestmark = pytest.mark.gpu

SHAPES = [
    pytest.param(dict(hidden=1536, hq=12, hkv=2, hd=128, inter=8960), id="1p5b"),
    pytest.param(dict(hidden=896, hq=14, hkv=2, hd=64, inter=4864), id="0p5b"),
    pytest.param(dict(hidden=256, hq=4, hkv=2, hd=64, inter=512), id="tiny"),
]


def _rand(shape, scale, g):
    return (torch.randn(*shape, generator=g) * scale).to(torch.bfloat16)


class Layer:
    def __init__(self, s, seed, gpu):
        g = torch.Generator().manual_seed(seed)
        H, I = s["hidden"], s["inter"]
        qd, kvd = s["hq"] * s["hd"], s["hkv"] * s["hd"]
        self.w_o = _rand((H, qd), 0.03, g).to(gpu)
        self.post = (1 + 0.1 * torch.randn(H, generator=g)).to(torch.bfloat16).to(gpu)
        self.w_gu = _rand((2 * I, H), 0.05, g).to(gpu)
        self.w_down = _rand((H, I), 0.03, g).to(gpu)
        self.in_norm = (1 + 0.1 * torch.randn(H, generator=g)).to(torch.bfloat16).to(gpu)
        self.w_qkv = _rand((qd + 2 * kvd, H), 0.03, g).to(gpu)
        self.b_qkv = _rand((qd + 2 * kvd,), 0.03, g).to(gpu)


def _setup(s, kv_len, max_kv, gpu, seed=0):
    g = torch.Generator().manual_seed(seed)
    hq, hkv, hd = s["hq"], s["hkv"], s["hd"]
    ctx = C.make_attention_ctx(hq, hkv, hd)
    q = torch.randn(1, hq, hd, generator=g).to(torch.bfloat16).to(gpu)
    k = torch.randn(max_kv, hkv, hd, generator=g).to(torch.bfloat16).to(gpu)
    v = torch.randn(max_kv, hkv, hd, generator=g).to(torch.bfloat16).to(gpu)
    d_len = torch.tensor([kv_len], dtype=torch.int32, device=gpu)
    ws = torch.zeros(C.load().efm_attention_decode_workspace_bytes(ctx, max_kv), dtype=torch.uint8, device=gpu)
    C.call("efm_decode_attention_partials", ctx, ptr(q), ptr(k), ptr(v), ptr(d_len), max_kv, ptr(ws), ws.numel(),
           stream())
    r = torch.randn(1, s["hidden"], generator=g).to(torch.bfloat16).to(gpu)
    return ctx, (q, k, v), d_len, ws, r


def _unfused(s, ctx, d_len, max_kv, ws, r_in, L, last, eps=1e-6):
    gpu = r_in.device
    H, I = s["hidden"], s["inter"]
    qd, kvd = s["hq"] * s["hd"], s["hkv"] * s["hd"]
    a = torch.empty(1, H, dtype=torch.bfloat16, device=gpu)
    C.call("efm_decode_attention_merge_o_proj", ctx, ptr(d_len), max_kv, ptr(ws), ws.numel(), ptr(L.w_o), H, ptr(a),
           stream())
    r_mid = torch.empty_like(a)
    mid = torch.empty(1, I, dtype=torch.bfloat16, device=gpu)
    C.call("efm_decode_norm_gate_up_swiglu", H, I, eps, ptr(a), ptr(r_in), ptr(r_mid), ptr(L.post), ptr(L.w_gu),
           ptr(mid), stream())
    h = torch.empty(1, H, dtype=torch.bfloat16, device=gpu)
    C.call("efm_linear", 1, I, H, ptr(mid), ptr(L.w_down), None, ptr(h), C.EFM_DTYPE_BF16, stream())
    out = {"a": a, "r_mid": r_mid, "mid": mid, "h": h}
    if not last:
        r_next = torch.empty_like(a)
        qn = torch.empty(1, qd, dtype=torch.bfloat16, device=gpu)
        kc = torch.zeros(max_kv, kvd, dtype=torch.bfloat16, device=gpu)
        vc = torch.zeros_like(kc)
        C.call("efm_decode_norm_qkv", H, qd, kvd, eps, ptr(h), ptr(r_mid), ptr(r_next), ptr(L.in_norm),
               ptr(L.w_qkv), ptr(L.b_qkv), ptr(qn), ptr(kc), ptr(vc), ptr(d_len), stream())
        out.update(r_next=r_next, q=qn, kc=kc, vc=vc)
    torch.cuda.synchronize()
    return out


def _chain(s, ctx, d_len, max_kv, ws, r_in, L, last, cws, eps=1e-6):
    gpu = r_in.device
    H, I = s["hidden"], s["inter"]
    qd, kvd = s["hq"] * s["hd"], s["hkv"] * s["hd"]
    r_out = torch.full((1, H), 7.0, dtype=torch.bfloat16, device=gpu)
    h_out = torch.full((1, H), 7.0, dtype=torch.bfloat16, device=gpu)
    qn = torch.full((1, qd), 7.0, dtype=torch.bfloat16, device=gpu)
    kc = torch.zeros(max_kv, kvd, dtype=torch.bfloat16, device=gpu)
    vc = torch.zeros_like(kc)
    desc = C.DecodeChainLayer(ptr(L.w_o), ptr(L.post), ptr(L.w_gu), ptr(L.w_down),
                              None if last else ptr(L.in_norm), None if last else ptr(L.w_qkv),
                              None if last else ptr(L.b_qkv), None if last else ptr(qn),
                              None if last else ptr(kc), None if last else ptr(vc))
    C.call("efm_decode_layer_chain", ctx, H, I, eps, desc, ptr(d_len), max_kv, ptr(ws), ws.numel(), ptr(r_in),
           ptr(r_out), ptr(h_out) if last else None, ptr(cws), cws.numel(), stream())
    torch.cuda.synchronize()
    C.call("efm_decode_chain_status", ptr(cws), H, I, stream())
    return {"r_out": r_out, "h": h_out, "q": qn, "kc": kc, "vc": vc}


def _chain_ws(s, gpu):
    n = C.load().efm_decode_chain_workspace_bytes(s["hidden"], s["inter"])
    return torch.zeros(n, dtype=torch.uint8, device=gpu)


@pytest.mark.parametrize("s", SHAPES)
@pytest.mark.parametrize("kv_len", [1, 300, 767])
def test_chain_bit_exact_vs_unfused(gpu, s, kv_len):
    max_kv = 768
    ctx = C.make_attention_ctx(s["hq"], s["hkv"], s["hd"])
    C.call("efm_decode_chain_supported", ctx, s["hidden"], s["inter"], max_kv)
    cws = _chain_ws(s, gpu)
    L = Layer(s, seed=1, gpu=gpu)
    ctx, _, d_len, ws, r_in = _setup(s, kv_len, max_kv, gpu)
    ref = _unfused(s, ctx, d_len, max_kv, ws, r_in, L, last=False)
    got = _chain(s, ctx, d_len, max_kv, ws, r_in, L, last=False, cws=cws)
    assert torch.equal(got["r_out"], ref["r_next"]), "residual r_{l+1}"
    assert torch.equal(got["q"], ref["q"]), "q of the next layer"
    assert torch.equal(got["kc"], ref["kc"]) and torch.equal(got["vc"], ref["vc"]), "next layer's KV slot"
    assert got["kc"][kv_len - 1].abs().sum() > 0 and got["kc"][kv_len:].abs().sum() == 0


@pytest.mark.parametrize("s", SHAPES)
def test_chain_last_layer_bit_exact(gpu, s):
    max_kv = 512
    cws = _chain_ws(s, gpu)
    L = Layer(s, seed=2, gpu=gpu)
    ctx, _, d_len, ws, r_in = _setup(s, 200, max_kv, gpu, seed=3)
    ref = _unfused(s, ctx, d_len, max_kv, ws, r_in, L, last=True)
    got = _chain(s, ctx, d_len, max_kv, ws, r_in, L, last=True, cws=cws)
    assert torch.equal(got["h"], ref["h"]), "down_proj output"
    assert torch.equal(got["r_out"], ref["r_mid"]), "post-attention residual"


def test_chain_repeated_launches_and_oracle(gpu):
    """Eight launches in a row on one workspace (the tag advances each time), each with
    new inputs; every result equals the unfused path, and the first also the oracle."""
    s = dict(hidden=1536, hq=12, hkv=2, hd=128, inter=8960)
    max_kv = 1024
    cws = _chain_ws(s, gpu)
    for it in range(8):
        L = Layer(s, seed=10 + it, gpu=gpu)
        kv_len = 100 + 111 * it
        ctx, (q, k, v), d_len, ws, r_in = _setup(s, kv_len, max_kv, gpu, seed=20 + it)
        ref = _unfused(s, ctx, d_len, max_kv, ws, r_in, L, last=(it % 3 == 2))
        got = _chain(s, ctx, d_len, max_kv, ws, r_in, L, last=(it % 3 == 2), cws=cws)
        if it % 3 == 2:
            assert torch.equal(got["h"], ref["h"]) and torch.equal(got["r_out"], ref["r_mid"]), f"launch {it}"
        else:
            assert torch.equal(got["q"], ref["q"]) and torch.equal(got["r_out"], ref["r_next"]), f"launch {it}"
        if it == 0:
            eps = 1e-6
            att = O.attention_decode(q.cpu(), k.cpu(), v.cpu(), kv_len, O.AttnCtx(12, 2, 128)).reshape(1, -1)
            a = O.linear(att, L.w_o.cpu())
            x2, r_mid = O.fused_add_rms_norm(a, r_in.cpu(), L.post.cpu(), eps)
            h = O.linear(O.gate_up_swiglu(x2, L.w_gu.cpu()), L.w_down.cpu())
            x, r_next = O.fused_add_rms_norm(h, r_mid, L.in_norm.cpu(), eps)
            qkv = O.linear(x, L.w_qkv.cpu(), L.b_qkv.cpu())
            # bf16 roundings of the 8960 SwiGLU outputs differ by an ulp here and there
            # between any two summation orders; |h| ~ 8 makes that ~0.06 absolute, so
            # the tolerance scales with the vector (2 % of its largest element)
            for name, g_, r_ in (("r_next", got["r_out"], r_next), ("q", got["q"], qkv[:, :1536])):
                tol = 2e-2 * float(r_.float().abs().max())
                assert_close_bf16(g_, r_, rtol=2e-2, atol=tol, what=f"{name} vs oracle")


def test_chain_rejects_unsupported(gpu):
    ctx = C.make_attention_ctx(28, 4, 128)
    with pytest.raises(C.EfmError):
        C.call("efm_decode_chain_supported", ctx, 3584, 18944, 1024)       # 7B rows exceed the chain
    ctx = C.make_attention_ctx(12, 2, 128)
    with pytest.raises(C.EfmError):
        C.call("efm_decode_chain_supported", ctx, 1536, 8960, 4096)        # > 8 attention splits
    C.call("efm_decode_chain_supported", ctx, 1536, 8960, 1024)
