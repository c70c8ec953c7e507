"""GPU tests of the fused decode front half (efm_decode_norm_qkv_attention).

It must equal, bit for bit, the unfused pair it replaces, efm_decode_norm_qkv followed by
efm_decode_attention_partials on the rotated cache (k_already_prerotated =
EFM_K_PREROTATED_EXCEPT_NEWEST), whose kernels are pinned to the oracle in
test_gpu_ops.py: the residual output, every cache row (V and the rotated newest K in slot
L-1, nothing else touched, NaN rows past L kept) and the attention split partials. Checked
for the 1.5B, VL-3B text and 7B head layouts, at split boundaries, over many launches in a
row on one sync workspace (the launch tag advances each time) and under HIP graph replay;
the bounded wait forced to give up from the host is reported once and later launches
are exact again."""
import pytest
import torch

import efm_capi as C
from _util import ptr, stream

pytestmark = pytest.mark.gpu

SHAPES = {
    "1p5b": dict(hidden=1536, hq=12, hkv=2, hd=128, max_kv=768),
    "vl3b": dict(hidden=2048, hq=16, hkv=2, hd=128, max_kv=512),
    "7b": dict(hidden=3584, hq=28, hkv=4, hd=128, max_kv=1024),
}


def _ctx(s):
    ctx = C.make_attention_ctx(s["hq"], s["hkv"], s["hd"])
    ctx.k_already_prerotated = C.EFM_K_PREROTATED_EXCEPT_NEWEST
    return ctx


class Case:
    def __init__(self, s, L, seed, gpu):
        g = torch.Generator().manual_seed(seed)
        H, qd, kvd = s["hidden"], s["hq"] * s["hd"], s["hkv"] * s["hd"]
        n = qd + 2 * kvd
        self.W = (torch.randn(n, H, generator=g) * 0.03).to(torch.bfloat16).to(gpu)
        self.b = (torch.randn(n, generator=g) * 0.03).to(torch.bfloat16).to(gpu)
        self.nw = (1 + 0.1 * torch.randn(H, generator=g)).to(torch.bfloat16).to(gpu)
        self.h = torch.randn(1, H, generator=g).to(torch.bfloat16).to(gpu)
        self.r = torch.randn(1, H, generator=g).to(torch.bfloat16).to(gpu)
        kc = torch.full((s["max_kv"], kvd), float("nan"), dtype=torch.bfloat16)
        vc = torch.full((s["max_kv"], kvd), float("nan"), dtype=torch.bfloat16)
        kc[:L] = torch.randn(L, kvd, generator=g).to(torch.bfloat16)   # rows < L-1: rotated keys
        vc[:L] = torch.randn(L, kvd, generator=g).to(torch.bfloat16)   # row L-1: overwritten
        self.kc, self.vc = kc.to(gpu), vc.to(gpu)
        self.d_len = torch.tensor([L], dtype=torch.int32, device=gpu)


def _bits(t):
    return t.view(torch.int16) if t.dtype == torch.bfloat16 else t.view(torch.int32)


def _unfused(s, ctx, c, layer0, ws_bytes, eps=1e-6):
    gpu = c.h.device
    qd, kvd = s["hq"] * s["hd"], s["hkv"] * s["hd"]
    kc, vc = c.kc.clone(), c.vc.clone()
    q = torch.empty(1, qd, dtype=torch.bfloat16, device=gpu)
    r_out = torch.empty_like(c.h)
    ws = torch.zeros(ws_bytes, dtype=torch.uint8, device=gpu)
    C.call("efm_decode_norm_qkv", s["hidden"], qd, kvd, eps, ptr(c.h), None if layer0 else ptr(c.r), ptr(r_out),
           ptr(c.nw), ptr(c.W), ptr(c.b), ptr(q), ptr(kc), ptr(vc), ptr(c.d_len), stream())
    C.call("efm_decode_attention_partials", ctx, ptr(q), ptr(kc), ptr(vc), ptr(c.d_len), s["max_kv"], ptr(ws),
           ws.numel(), stream())
    return r_out, kc, vc, ws


def _fused(s, ctx, c, layer0, ws_bytes, sync, eps=1e-6):
    kc, vc = c.kc.clone(), c.vc.clone()
    r_out = torch.empty_like(c.h)
    ws = torch.zeros(ws_bytes, dtype=torch.uint8, device=c.h.device)
    C.call("efm_decode_norm_qkv_attention", ctx, s["hidden"], eps, ptr(c.h), None if layer0 else ptr(c.r),
           ptr(r_out), ptr(c.nw), ptr(c.W), ptr(c.b), ptr(kc), ptr(vc), ptr(c.d_len), s["max_kv"], ptr(ws),
           ws.numel(), ptr(sync), sync.numel(), stream())
    return r_out, kc, vc, ws


def _sync_ws(s, gpu):
    n = C.load().efm_decode_qkv_attention_sync_bytes(s["hq"] * s["hd"], s["hkv"] * s["hd"])
    return torch.zeros(n, dtype=torch.uint8, device=gpu)


def _assert_same(ref, got, what):
    for name, a, b in zip(("residual", "K cache", "V cache", "attention partials"), ref, got):
        assert torch.equal(_bits(a), _bits(b)), f"{what}: {name} differs"


@pytest.mark.parametrize("shape,L", [("1p5b", 1), ("1p5b", 128), ("1p5b", 129), ("1p5b", 513), ("1p5b", 768),
                                     ("vl3b", 77), ("vl3b", 512), ("7b", 1), ("7b", 1000)])
@pytest.mark.parametrize("layer0", [False, True])
def test_fused_bit_exact_vs_unfused(gpu, shape, L, layer0):
    s = SHAPES[shape]
    ctx = _ctx(s)
    C.call("efm_decode_norm_qkv_attention_supported", ctx, s["hidden"], s["max_kv"])
    ws_bytes = C.load().efm_attention_decode_workspace_bytes(ctx, s["max_kv"])
    c = Case(s, L, seed=L + 7 * layer0, gpu=gpu)
    sync = _sync_ws(s, gpu)
    ref = _unfused(s, ctx, c, layer0, ws_bytes)
    got = _fused(s, ctx, c, layer0, ws_bytes, sync)
    torch.cuda.synchronize()
    _assert_same(ref, got, f"{shape} L={L}")
    kvd = s["hkv"] * s["hd"]
    assert not torch.isnan(got[1][L - 1].float()).any() and torch.isnan(got[1][L:].float()).all()
    assert torch.equal(_bits(got[1][: L - 1]), _bits(c.kc[: L - 1])), "rows before the newest must not change"
    assert got[3].abs().sum() > 0
    C.call("efm_decode_qkv_attention_status", ptr(sync), stream())
    assert kvd == got[2].shape[1]


def test_fused_many_launches_one_sync_workspace(gpu):
    """Twenty launches on one sync workspace with new inputs and lengths each time (the
    epoch advances per launch; a stale word of the previous launch must never pass)."""
    s = SHAPES["1p5b"]
    ctx = _ctx(s)
    ws_bytes = C.load().efm_attention_decode_workspace_bytes(ctx, s["max_kv"])
    sync = _sync_ws(s, gpu)
    for it in range(20):
        L = 1 + (it * 97) % s["max_kv"]
        c = Case(s, L, seed=100 + it, gpu=gpu)
        ref = _unfused(s, ctx, c, it % 5 == 0, ws_bytes)
        got = _fused(s, ctx, c, it % 5 == 0, ws_bytes, sync)
        torch.cuda.synchronize()
        _assert_same(ref, got, f"launch {it} L={L}")
    C.call("efm_decode_qkv_attention_status", ptr(sync), stream())
    epoch = int(sync[:4].view(torch.int32).item())
    done = int(sync[4:8].view(torch.int32).item())
    assert epoch == 20 and done == 0


def test_fused_graph_replay(gpu):
    """Three fused launches captured in one HIP graph (three layers of one step), replayed
    five times with eager work in between; every replay equals the unfused results."""
    s = SHAPES["1p5b"]
    ctx = _ctx(s)
    ws_bytes = C.load().efm_attention_decode_workspace_bytes(ctx, s["max_kv"])
    sync = _sync_ws(s, gpu)
    cases = [Case(s, 300 + 100 * i, seed=40 + i, gpu=gpu) for i in range(3)]
    refs = [_unfused(s, ctx, c, i == 0, ws_bytes) for i, c in enumerate(cases)]
    torch.cuda.synchronize()
    bufs = []
    for c in cases:
        bufs.append(dict(kc=torch.empty_like(c.kc), vc=torch.empty_like(c.vc), r=torch.empty_like(c.h),
                         ws=torch.zeros(ws_bytes, dtype=torch.uint8, device=gpu)))
    st = torch.cuda.Stream()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=st, capture_error_mode="thread_local"):
        for i, (c, b) in enumerate(zip(cases, bufs)):
            C.call("efm_decode_norm_qkv_attention", ctx, s["hidden"], 1e-6, ptr(c.h), None if i == 0 else ptr(c.r),
                   ptr(b["r"]), ptr(c.nw), ptr(c.W), ptr(c.b), ptr(b["kc"]), ptr(b["vc"]), ptr(c.d_len), s["max_kv"],
                   ptr(b["ws"]), ws_bytes, ptr(sync), sync.numel(), st.cuda_stream)
    for rep in range(5):
        for c, b in zip(cases, bufs):
            b["kc"].copy_(c.kc)
            b["vc"].copy_(c.vc)
            b["ws"].zero_()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        for i, (ref, b) in enumerate(zip(refs, bufs)):
            _assert_same(ref, (b["r"], b["kc"], b["vc"], b["ws"]), f"replay {rep} layer {i}")
    C.call("efm_decode_qkv_attention_status", ptr(sync), stream())


def test_forced_wait_timeout_reported_then_recovers(gpu, knob):
    """The attention splits' bounded wait, forced to give up from the host
    (EFM_KNOB_FRONT_WAIT_TIMEOUT: they wait for a tag that no projected word carries, with
    a 64-poll limit, so every kernel still drains): three such launches flag the sync
    workspace, the status call reports EFM_ERR_DEVICE once, clears the flag and steps the
    epoch past every tag already written, and the launches after it, on the same sync
    workspace, are bit-exact with the unfused pair again."""
    s = SHAPES["1p5b"]
    ctx = _ctx(s)
    ws_bytes = C.load().efm_attention_decode_workspace_bytes(ctx, s["max_kv"])
    sync = _sync_ws(s, gpu)
    c = Case(s, 300, seed=5, gpu=gpu)
    ref = _unfused(s, ctx, c, False, ws_bytes)
    knob(C.EFM_KNOB_FRONT_WAIT_TIMEOUT, 1)
    bad = [_fused(s, ctx, c, False, ws_bytes, sync) for _ in range(3)]
    torch.cuda.synchronize()
    words = sync[:12].view(torch.int32).tolist()    # epoch, done, abort
    assert words == [3, 0, 1], f"sync header after three timed-out launches: {words}"
    # the splits went on with zeros for the query: their partials are not the real ones
    assert not torch.equal(_bits(bad[-1][3]), _bits(ref[3]))
    # the GEMV half never waits: the residual and the V row are right all the same
    assert torch.equal(_bits(bad[-1][0]), _bits(ref[0])) and torch.equal(_bits(bad[-1][2]), _bits(ref[2]))
    with pytest.raises(C.EfmError, match="timed out") as err:
        C.call("efm_decode_qkv_attention_status", ptr(sync), stream())
    assert err.value.code == C.EFM_ERR_DEVICE
    assert sync[:12].view(torch.int32).tolist() == [4, 0, 0]
    C.call("efm_decode_qkv_attention_status", ptr(sync), stream())   # reported once
    knob(C.EFM_KNOB_FRONT_WAIT_TIMEOUT, 0)
    for it in range(3):
        got = _fused(s, ctx, c, False, ws_bytes, sync)
        torch.cuda.synchronize()
        _assert_same(ref, got, f"launch {it} after the time-out")
    C.call("efm_decode_qkv_attention_status", ptr(sync), stream())
    assert sync[:12].view(torch.int32).tolist() == [7, 0, 0]


def test_fused_supported_limits(gpu):
    ok = _ctx(SHAPES["1p5b"])
    C.call("efm_decode_norm_qkv_attention_supported", ok, 1536, 768)
    C.call("efm_decode_norm_qkv_attention_supported", ok, 1536, 8192)      # 64 splits per KV head
    bad = []
    c = _ctx(SHAPES["1p5b"])
    bad.append((c, 1536, 16384))                                             # 256 attention workgroups
    bad.append((c, 8192, 768))                                               # hidden > 4096
    c2 = C.make_attention_ctx(12, 2, 128)                                    # un-rotated cache
    bad.append((c2, 1536, 768))
    c3 = C.make_attention_ctx(14, 2, 64)
    c3.k_already_prerotated = C.EFM_K_PREROTATED_EXCEPT_NEWEST               # head_dim 64
    bad.append((c3, 896, 1024))
    for ctx, hidden, mk in bad:
        with pytest.raises(C.EfmError):
            C.call("efm_decode_norm_qkv_attention_supported", ctx, hidden, mk)
    s = SHAPES["1p5b"]
    sync = _sync_ws(s, gpu)
    c = Case(s, 10, seed=1, gpu=gpu)
    ws_bytes = C.load().efm_attention_decode_workspace_bytes(ok, s["max_kv"])
    ws = torch.zeros(ws_bytes, dtype=torch.uint8, device=gpu)
    r_out = torch.empty_like(c.h)
    with pytest.raises(C.EfmError):   # sync workspace too small
        C.call("efm_decode_norm_qkv_attention", ok, s["hidden"], 1e-6, ptr(c.h), ptr(c.r), ptr(r_out), ptr(c.nw),
               ptr(c.W), ptr(c.b), ptr(c.kc), ptr(c.vc), ptr(c.d_len), s["max_kv"], ptr(ws), ws_bytes, ptr(sync),
               16, stream())
