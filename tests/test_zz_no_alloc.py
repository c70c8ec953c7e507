"""efm_attention_decode_noalloc: decode attention whose split partials live in the
library's own device array instead of a caller workspace. Its results must equal
efm_attention_decode's (same kernels) bit for bit, call after call, also when a later call
is smaller than an earlier one (the array keeps the last call's contents)."""
import pytest
import torch

import efm_capi as C
from oracle import efm_oracle as O
from _util import assert_close_bf16, ptr, stream


def _with_workspace(ctx, q, k, v, kv_len, d_len, max_kv):
    bound = max_kv if d_len is not None else kv_len
    ws = torch.zeros(C.load().efm_attention_decode_workspace_bytes(ctx, bound), dtype=torch.uint8, device=q.device)
    o = torch.empty_like(q)
    C.call("efm_attention_decode", ctx, ptr(q), ptr(k), ptr(v), ptr(o), kv_len, ptr(d_len), max_kv, ptr(ws),
           ws.numel(), stream())
    return o


def _noalloc(ctx, q, k, v, kv_len, d_len, max_kv):
    o = torch.full_like(q, float("nan"))
    C.call("efm_attention_decode_noalloc", ctx, ptr(q), ptr(k), ptr(v), ptr(o), kv_len, ptr(d_len), max_kv, stream())
    return o


# (heads, kv heads, head_dim, kv_len, max_kv or None): large first, then a smaller call
CASES = [
    [(28, 4, 128, 16385, 16513), (12, 2, 128, 300, None)],
    [(12, 2, 128, 2048, None), (14, 2, 64, 77, 1025)],
    [(16, 2, 128, 1344, 1500), (16, 2, 128, 1, 1)],
]


@pytest.mark.gpu
@pytest.mark.parametrize("seq", CASES, ids=["7b16k_then_1p5b", "1p5b_then_0p5b_graphlike", "3b_then_len1"])
def test_noalloc_matches_workspace_entry_point(gpu, seq):
    for i, (hq, hkv, hd, kv_len, max_kv) in enumerate(seq):
        torch.manual_seed(kv_len * 7 + hq)
        rows = max_kv or kv_len
        q = torch.randn(1, hq, hd, dtype=torch.bfloat16, device=gpu)
        k = torch.randn(rows, hkv, hd, dtype=torch.bfloat16, device=gpu)
        v = torch.randn(rows, hkv, hd, dtype=torch.bfloat16, device=gpu)
        d_len = torch.tensor([kv_len], dtype=torch.int32, device=gpu) if max_kv else None
        ctx = C.make_attention_ctx(hq, hkv, hd)
        ref = _with_workspace(ctx, q, k, v, kv_len, d_len, max_kv or 0)
        got = _noalloc(ctx, q, k, v, kv_len, d_len, max_kv or 0)
        again = _noalloc(ctx, q, k, v, kv_len, d_len, max_kv or 0)
        torch.cuda.synchronize()
        assert torch.equal(got, ref), f"call {i}: noalloc differs from efm_attention_decode"
        assert torch.equal(again, ref), f"call {i}: repeated noalloc call differs"
        if kv_len <= 2048:
            exp = O.attention_decode(q.cpu(), k[:kv_len].cpu(), v[:kv_len].cpu(), kv_len, O.AttnCtx(hq, hkv, hd))
            assert_close_bf16(got.reshape(1, hq, hd), exp, what=f"call {i} vs oracle")


@pytest.mark.gpu
def test_noalloc_captured_in_a_graph_matches_workspace_entry_point(gpu):
    """After efm_init, noalloc calls of two shapes (the C2 heads over a 768-row cache with
    a device-side length, then the 0.5B heads) are captured into one graph and replayed
    three times, with eager work and synchronisations between the replays and the length
    changed on the device; every replay equals efm_attention_decode's eager result bit for
    bit."""
    assert C.load().efm_init() == C.EFM_OK
    torch.manual_seed(5)
    shapes = [(12, 2, 128, 768), (14, 2, 64, 1100)]
    bufs = []
    for hq, hkv, hd, rows in shapes:
        q = torch.randn(1, hq, hd, dtype=torch.bfloat16, device=gpu)
        k = torch.randn(rows, hkv, hd, dtype=torch.bfloat16, device=gpu)
        v = torch.randn(rows, hkv, hd, dtype=torch.bfloat16, device=gpu)
        d_len = torch.tensor([rows // 2], dtype=torch.int32, device=gpu)
        bufs.append((C.make_attention_ctx(hq, hkv, hd), q, k, v, d_len, rows, torch.empty_like(q)))
    s = torch.cuda.Stream()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s, capture_error_mode="thread_local"):
        for ctx, q, k, v, d_len, rows, o in bufs:
            C.call("efm_attention_decode_noalloc", ctx, ptr(q), ptr(k), ptr(v), ptr(o), 0, ptr(d_len), rows,
                   s.cuda_stream)
    for rep, length_frac in enumerate((0.5, 0.9, 0.25)):
        for ctx, q, k, v, d_len, rows, o in bufs:
            d_len.fill_(max(1, int(rows * length_frac)))
            o.fill_(float("nan"))
        torch.randn(1 << 20, device=gpu).sum()   # eager work between replays
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        for i, (ctx, q, k, v, d_len, rows, o) in enumerate(bufs):
            ref = _with_workspace(ctx, q, k, v, 0, d_len, rows)
            torch.cuda.synchronize()
            assert torch.equal(o, ref), f"replay {rep}, call {i}: captured noalloc differs from efm_attention_decode"


def test_noalloc_rejects_shapes_beyond_its_array():
    """A shape whose split partials need more than the library's array is refused on the
    host before anything is launched (no GPU needed)."""
    lib = C.load()
    ctx = C.make_attention_ctx(8192, 1024, 128)   # 1024 KV heads, group 8: 4 MiB of partials
    assert lib.efm_attention_decode_workspace_bytes(ctx, 64) > C.EFM_ATTENTION_DECODE_NOALLOC_SCRATCH_BYTES
    rc = lib.efm_attention_decode_noalloc(ctx, 16, 16, 16, 16, 64, None, 0, None)
    assert rc == C.EFM_ERR_UNSUPPORTED and b"scratch" in lib.efm_last_error()
