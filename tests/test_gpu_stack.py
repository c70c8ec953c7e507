"""GPU tests of the whole-step persistent decode kernel (efm_decode_stack).

One launch runs every layer of a decode step. It must agree with the per-layer launch
sequence it replaces (efm_embedding_lookup, efm_decode_norm_qkv, efm_attention_decode on
the rotated cache, efm_linear o_proj, efm_decode_norm_gate_up_swiglu, efm_linear down),
whose kernels are pinned to the oracle in test_gpu_ops.py, to bf16 rounding: the two sum
every dot product in a different order. It is also checked against the oracle's logits
end to end, for rerun determinism, over many launches on one workspace (each launch tags
its hand-offs with a new epoch) and under HIP-graph replay."""
import pytest
import torch

import efm_capi as C
from oracle import efm_oracle as O
from _util import assert_close_bf16, ptr, stream

pytestmark = pytest.mark.gpu

EPS = 1e-6


class Model:
    """Random Qwen2.5-shaped decoder (fused weights of the oracle), per-layer K / V caches
    whose rows [0, L-1) hold keys rotated at their positions (the engine's cache), and the
    device layer table of efm_decode_stack."""

    def __init__(self, gpu, hidden, hq, hkv, inter, layers, vocab, max_kv, kv_len, seed, std=0.02):
        self.cfg = O.QwenConfig(hidden=hidden, layers=layers, heads=hq, kv_heads=hkv, head_dim=128, inter=inter,
                                vocab=vocab)
        self.w = O.fuse_weights(self.cfg, O.random_weights(self.cfg, seed=seed, std=std))
        self.wg = {k: v.to(gpu).contiguous() for k, v in self.w.items()}
        g = torch.Generator().manual_seed(seed + 1)
        self.k_raw = [torch.randn(max_kv, hkv, 128, generator=g).to(torch.bfloat16) for _ in range(layers)]
        self.v = [torch.randn(max_kv, hkv, 128, generator=g).to(torch.bfloat16) for _ in range(layers)]
        pos = torch.arange(max_kv)
        self.k_rot = [O.rope_llama(k, pos, 1.0e6).to(torch.bfloat16) for k in self.k_raw]
        self.max_kv, self.kv_len, self.gpu = max_kv, kv_len, gpu
        self.ctx = C.make_attention_ctx(hq, hkv, 128)
        self.ctx.k_already_prerotated = C.EFM_K_PREROTATED_EXCEPT_NEWEST

    def caches(self):
        """Fresh device caches: rows [0, L-1) rotated, row L-1 and beyond NaN (the step
        writes row L-1; rows past it must never be used)."""
        kc, vc = [], []
        for l in range(self.cfg.layers):
            k = self.k_rot[l].clone()
            v = self.v[l].clone()
            k[self.kv_len - 1:] = float("nan")
            v[self.kv_len - 1:] = float("nan")
            kc.append(k.to(self.gpu).contiguous())
            vc.append(v.to(self.gpu).contiguous())
        return kc, vc

    def table(self, kc, vc):
        rows = []
        for l in range(self.cfg.layers):
            w = self.wg
            rows.append([w[f"{l}.in_norm"].data_ptr(), w[f"{l}.qkv_w"].data_ptr(), w[f"{l}.qkv_b"].data_ptr(),
                         w[f"{l}.o_w"].data_ptr(), w[f"{l}.post_norm"].data_ptr(), w[f"{l}.gu_w"].data_ptr(),
                         w[f"{l}.down_w"].data_ptr(), kc[l].data_ptr(), vc[l].data_ptr()])
        return torch.tensor(rows, dtype=torch.int64, device=self.gpu)

    def workspace(self):
        c = self.cfg
        n = C.load().efm_decode_stack_workspace_bytes(self.ctx, c.hidden, c.inter, c.layers, self.max_kv)
        assert n > 0, C.load().efm_last_error()
        return torch.zeros(n, dtype=torch.uint8, device=self.gpu)

    def stack(self, token, kc, vc, ws, st=None):
        c = self.cfg
        tab = self.table(kc, vc)
        tok = torch.tensor([token], dtype=torch.int32, device=self.gpu)
        d_len = torch.tensor([self.kv_len], dtype=torch.int32, device=self.gpu)
        h = torch.full((1, c.hidden), float("nan"), dtype=torch.bfloat16, device=self.gpu)
        r = torch.full_like(h, float("nan"))
        C.call("efm_decode_stack", self.ctx, c.hidden, c.inter, c.layers, EPS, ptr(tab), ptr(self.wg["embed"]),
               c.vocab, ptr(tok), ptr(d_len), self.max_kv, ptr(h), ptr(r), ptr(ws), ws.numel(),
               stream() if st is None else st)
        torch.cuda.synchronize()
        C.call("efm_decode_stack_status", ptr(ws), stream())
        return h, r

    def unfused(self, token, kc, vc):
        """The per-layer launch sequence of the engine's unfused decode path."""
        c, w, gpu = self.cfg, self.wg, self.gpu
        H, I, QD, KVD = c.hidden, c.inter, c.heads * 128, c.kv_heads * 128
        tok = torch.tensor([token], dtype=torch.int32, device=gpu)
        d_len = torch.tensor([self.kv_len], dtype=torch.int32, device=gpu)
        h = torch.empty(1, H, dtype=torch.bfloat16, device=gpu)
        C.call("efm_embedding_lookup", 1, H, c.vocab, ptr(tok), ptr(w["embed"]), None, 0, -1, ptr(h), stream())
        r0 = torch.empty_like(h)
        r1 = torch.empty_like(h)
        ws = torch.zeros(C.load().efm_attention_decode_workspace_bytes(self.ctx, self.max_kv), dtype=torch.uint8,
                         device=gpu)
        for l in range(c.layers):
            q = torch.empty(1, QD, dtype=torch.bfloat16, device=gpu)
            C.call("efm_decode_norm_qkv", H, QD, KVD, EPS, ptr(h), None if l == 0 else ptr(r1), ptr(r0),
                   ptr(w[f"{l}.in_norm"]), ptr(w[f"{l}.qkv_w"]), ptr(w[f"{l}.qkv_b"]), ptr(q), ptr(kc[l]),
                   ptr(vc[l]), ptr(d_len), stream())
            o = torch.empty(1, QD, dtype=torch.bfloat16, device=gpu)
            C.call("efm_attention_decode", self.ctx, ptr(q), ptr(kc[l]), ptr(vc[l]), ptr(o), 0, ptr(d_len),
                   self.max_kv, ptr(ws), ws.numel(), stream())
            a = torch.empty(1, H, dtype=torch.bfloat16, device=gpu)
            C.call("efm_linear", 1, QD, H, ptr(o), ptr(w[f"{l}.o_w"]), None, ptr(a), C.EFM_DTYPE_BF16, stream())
            mid = torch.empty(1, I, dtype=torch.bfloat16, device=gpu)
            C.call("efm_decode_norm_gate_up_swiglu", H, I, EPS, ptr(a), ptr(r0), ptr(r1), ptr(w[f"{l}.post_norm"]),
                   ptr(w[f"{l}.gu_w"]), ptr(mid), stream())
            C.call("efm_linear", 1, I, H, ptr(mid), ptr(w[f"{l}.down_w"]), None, ptr(h), C.EFM_DTYPE_BF16,
                   stream())
        torch.cuda.synchronize()
        return h, r1

    def logits(self, h, r):
        c, w = self.cfg, self.wg
        x = h.clone()
        C.call("efm_fused_add_rms_norm", 1, c.hidden, EPS, ptr(x), ptr(r.clone()), ptr(w["final_norm"]), stream())
        out = torch.empty(1, c.vocab, dtype=torch.float32, device=self.gpu)
        C.call("efm_linear", 1, c.hidden, c.vocab, ptr(x), ptr(w["lm_head"]), None, ptr(out), C.EFM_DTYPE_F32,
               stream())
        torch.cuda.synchronize()
        return out[0]


def _close(got, ref, what, frac=2e-2):
    tol = frac * float(ref.float().abs().max())
    assert torch.isfinite(got.float()).all(), f"{what}: non-finite values"
    assert_close_bf16(got, ref, rtol=frac, atol=tol, what=what)


SHAPES = [
    pytest.param(dict(hidden=1536, hq=12, hkv=2, inter=8960, layers=4), id="1p5b_4layers"),
    pytest.param(dict(hidden=2048, hq=16, hkv=2, inter=11008, layers=3), id="3b_3layers"),
    pytest.param(dict(hidden=896, hq=7, hkv=1, inter=4864, layers=3), id="g7_896"),
]


@pytest.mark.parametrize("s", SHAPES)
@pytest.mark.parametrize("kv_len,max_kv", [(1, 768), (300, 768), (768, 768), (1500, 2048)])
def test_stack_matches_unfused_sequence(gpu, s, kv_len, max_kv):
    m = Model(gpu, vocab=1000, max_kv=max_kv, kv_len=kv_len, seed=kv_len + s["hidden"], **s)
    C.call("efm_decode_stack_supported", m.ctx, s["hidden"], s["inter"], s["layers"], max_kv)
    token = 123
    kc_r, vc_r = m.caches()
    h_ref, r_ref = m.unfused(token, kc_r, vc_r)
    kc, vc = m.caches()
    ws = m.workspace()
    h, r = m.stack(token, kc, vc, ws)
    _close(h, h_ref, "h (last layer down_proj)")
    _close(r, r_ref, "residual")
    for l in range(s["layers"]):
        # this step's K (rotated) and V rows; rows before it untouched
        _close(kc[l][kv_len - 1], kc_r[l][kv_len - 1], f"layer {l} newest K row")
        _close(vc[l][kv_len - 1], vc_r[l][kv_len - 1], f"layer {l} newest V row")
        assert torch.equal(kc[l][: kv_len - 1], kc_r[l][: kv_len - 1])
    # a second launch on the same workspace (new epoch) from the same caches repeats bit for bit
    kc2, vc2 = m.caches()
    h2, r2 = m.stack(token, kc2, vc2, ws)
    assert torch.equal(h2, h) and torch.equal(r2, r), "rerun differs"


def test_stack_logits_match_oracle(gpu):
    """Against the CPU oracle (un-rotated cache, RoPE on read): the step's logits after the
    final norm + LM head, and the greedy token (or a near tie)."""
    kv_len, max_kv = 200, 256
    m = Model(gpu, hidden=512, hq=4, hkv=2, inter=1024, layers=3, vocab=1000, max_kv=max_kv, kv_len=kv_len, seed=5,
              std=0.05)
    token = 77
    kc, vc = m.caches()
    ws = m.workspace()
    h, r = m.stack(token, kc, vc, ws)
    got = m.logits(h, r).cpu()
    orc = O.Qwen2Oracle(m.cfg, m.w, max_tokens=max_kv)
    st = orc.new_state()
    for l in range(m.cfg.layers):
        st.k[l][: kv_len - 1] = m.k_raw[l][: kv_len - 1]
        st.v[l][: kv_len - 1] = m.v[l][: kv_len - 1]
    st.length = kv_len - 1
    ref = orc.forward(st, torch.tensor([token], dtype=torch.int32))
    tol = 2e-2 * float(ref.abs().max())
    torch.testing.assert_close(got, ref, rtol=2e-2, atol=tol)
    gtok, rtok = int(got.argmax()), int(O.argmax_lowest(ref.unsqueeze(0))[0])
    assert gtok == rtok or float(ref[rtok] - ref[gtok]) < 0.05


def test_stack_many_launches_and_graph_replay(gpu):
    """Twenty eager launches on one workspace (the epoch advances every launch), then the
    launch captured in a HIP graph and replayed three times with eager launches between;
    every result equals the first."""
    m = Model(gpu, hidden=1536, hq=12, hkv=2, inter=8960, layers=2, vocab=1000, max_kv=768, kv_len=513, seed=9)
    ws = m.workspace()
    kc, vc = m.caches()
    h0, r0 = m.stack(5, kc, vc, ws)
    for it in range(20):
        kc, vc = m.caches()
        h, r = m.stack(5, kc, vc, ws)
        assert torch.equal(h, h0) and torch.equal(r, r0), f"launch {it}"
    c = m.cfg
    kc, vc = m.caches()
    tab = m.table(kc, vc)
    tok = torch.tensor([5], dtype=torch.int32, device=gpu)
    d_len = torch.tensor([m.kv_len], dtype=torch.int32, device=gpu)
    hg = torch.empty(1, c.hidden, dtype=torch.bfloat16, device=gpu)
    rg = torch.empty_like(hg)
    st = torch.cuda.Stream()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=st, capture_error_mode="thread_local"):
        C.call("efm_decode_stack", m.ctx, c.hidden, c.inter, c.layers, EPS, ptr(tab), ptr(m.wg["embed"]), c.vocab,
               ptr(tok), ptr(d_len), m.max_kv, ptr(hg), ptr(rg), ptr(ws), ws.numel(), st.cuda_stream)
    for rep in range(3):
        hg.fill_(float("nan"))
        graph.replay()
        torch.cuda.synchronize()
        C.call("efm_decode_stack_status", ptr(ws), stream())
        assert torch.equal(hg, h0) and torch.equal(rg, r0), f"replay {rep}"
        kc2, vc2 = m.caches()
        h, r = m.stack(5, kc2, vc2, ws)
        assert torch.equal(h, h0), f"eager launch after replay {rep}"


def test_stack_supported_limits(gpu):
    ctx = C.make_attention_ctx(12, 2, 128)
    with pytest.raises(C.EfmError):
        C.call("efm_decode_stack_supported", ctx, 1536, 8960, 28, 1024)   # rotated cache required
    ctx.k_already_prerotated = C.EFM_K_PREROTATED_EXCEPT_NEWEST
    C.call("efm_decode_stack_supported", ctx, 1536, 8960, 28, 768)
    with pytest.raises(C.EfmError):
        C.call("efm_decode_stack_supported", ctx, 1536, 8960, 28, 16512)  # more than 16 splits per KV head
    ctx64 = C.make_attention_ctx(14, 2, 64)
    ctx64.k_already_prerotated = C.EFM_K_PREROTATED_EXCEPT_NEWEST
    with pytest.raises(C.EfmError):
        C.call("efm_decode_stack_supported", ctx64, 896, 4864, 24, 1024)  # head_dim 64
