"""CPU oracle for EdgeFM's single-request transformer hot path.

TEST INFRASTRUCTURE ONLY. This module is the checker that the HIP kernels are
compared against; only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline
leg may import it. The product path (edge-fm-x_amd/) never imports, links or
falls back to it.

It restates, on the CPU with PyTorch (bf16 storage, fp32 arithmetic), the operators
of the EdgeFM reference with the reference's rounding points:

* RMSNorm / fused add + RMSNorm — src/operators/norm_op.cu:20-106 (FlashInfer
  norm::RMSNorm / FusedAddRMSNorm); test closed forms
  tests/operators/test_norm_sampler.py:62-65,82-96.
* Linear — cuBLASLt y = x W^T (+b), fp32 accumulate (src/operators/linear_impl.cu:
  315-480); closed form tests/operators/test_decode_linear.py:161-181.
* SiLU-and-mul on [up; gate] — src/operators/activation_op.cu:18-76,
  tests/operators/test_fused_gate_up_activation.py:118-128.
* RoPE-Llama (rotate-half pairs (d, d+hd/2)) — src/operators/attention_op.cu:327-371;
  M-RoPE — src/layers/attention.cu:17-72.
* Decode / prefill attention semantics — src/operators/attention_op.cu:1345-1466
  (FlashInfer single_decode/single_prefill with ROPE_LLAMA, sm_scale 1/sqrt(hd)).
* Embedding with custom-embedding insertion — src/layers/embed_head.cu:63-132.
* Greedy argmax, ties to the lowest index — src/layers/sampler.cu:21-26.
* Qwen2.5 forward (op order, residual flow, fused [Q;K;V] / [up;gate] layouts, tied
  LM head, LM head on the last prefill row) — src/models/qwen2_5/qwen2_5.cpp:534-930,
  src/layers/linear.cu:1629-1785,1923-1943,2239-2286.
* Decode KV-slot / length bookkeeping — decode_runtime_kernels.cu:40-150,
  src/engine/tasks/token_generation/scheduler.cpp:123-134.

Parity pins for every function live in tests/test_oracle.py (closed forms, library
routines such as HF transformers' rotary embedding and Qwen2 model, brute force on
tiny inputs, invariants). The SageAttention-style int8 path and the temperature /
top-p sampler have no reference implementation; they are pinned by exact integer
restatement and by independent library routines respectively (see their docstrings).
"""
from __future__ import annotations

import math
from dataclasses import dataclass, field

import numpy as np
import torch

BF16 = torch.bfloat16
F32 = torch.float32


def bf(x: torch.Tensor) -> torch.Tensor:
    """Round to bf16 (round-to-nearest-even) and return as fp32."""
    return x.to(BF16).to(F32)


# ---------------------------------------------------------------------------------
# Norms, linear, activation
# ---------------------------------------------------------------------------------
def rms_norm(x: torch.Tensor, w: torch.Tensor, eps: float) -> torch.Tensor:
    """out = bf16((x * rsqrt(mean(x^2) + eps)) * w), fp32 math (norm_op.cu:20-60)."""
    xf = x.to(F32)
    inv = 1.0 / torch.sqrt(xf.pow(2).mean(dim=-1, keepdim=True) + eps)
    return ((xf * inv) * w.to(F32)).to(BF16)


def fused_add_rms_norm(x: torch.Tensor, residual: torch.Tensor, w: torch.Tensor, eps: float):
    """s = x + residual (fp32); residual' = bf16(s); out = RMSNorm of the fp32 s
    (norm_op.cu:62-106, FlashInfer FusedAddRMSNorm). Returns (out, residual')."""
    s = x.to(F32) + residual.to(F32)
    inv = 1.0 / torch.sqrt(s.pow(2).mean(dim=-1, keepdim=True) + eps)
    return ((s * inv) * w.to(F32)).to(BF16), s.to(BF16)


def linear(x: torch.Tensor, w: torch.Tensor, b: torch.Tensor | None = None, out_f32: bool = False) -> torch.Tensor:
    """y = x W^T (+ b) with fp32 accumulation; bf16 or fp32 output (linear_impl.cu:408-479)."""
    y = x.to(F32) @ w.to(F32).t()
    if b is not None:
        y = y + b.to(F32)
    return y if out_f32 else y.to(BF16)


def silu(x: torch.Tensor) -> torch.Tensor:
    """silu(x) = x / (1 + exp(-x)) (activation_op.cu:18-19)."""
    return x / (1.0 + torch.exp(-x))


def act_and_mul(x: torch.Tensor, up_first: bool = True) -> torch.Tensor:
    """out = bf16(silu(gate) * up) over rows laid out [up | gate] (up_first) or
    [gate | up] (activation_op.cu:36-76)."""
    h = x.shape[-1] // 2
    a, b = x[..., :h].to(F32), x[..., h:].to(F32)
    up, gate = (a, b) if up_first else (b, a)
    return (silu(gate) * up).to(BF16)


def gate_up_swiglu(x: torch.Tensor, w_up_gate: torch.Tensor) -> torch.Tensor:
    """Two-stage MLP front half: u, g = split(bf16(x [up; gate]^T)); bf16(silu(g) * u)
    (src/layers/gated_mlp.cu:19-67 with activation layout kUpGate)."""
    return act_and_mul(linear(x, w_up_gate), up_first=True)


# ---------------------------------------------------------------------------------
# Rotary embeddings
# ---------------------------------------------------------------------------------
def rope_inv_freq(head_dim: int, theta: float, rope_scale: float = 1.0) -> torch.Tensor:
    """inv_freq[d] = fp32((1/rope_scale) / theta^(2d/hd)), evaluated in float64 and
    rounded once (attention_op.cu:363-364)."""
    d = np.arange(head_dim // 2, dtype=np.float64)
    return torch.from_numpy((np.exp(-(2.0 * d / head_dim) * np.log(float(theta))) / float(rope_scale)).astype(np.float32))


def rope_angles(pos: torch.Tensor, head_dim: int, theta: float, rope_scale: float = 1.0) -> torch.Tensor:
    """angle[..., d] = fp32(pos) * inv_freq[d], an fp32 product; shape pos.shape + [hd/2]."""
    inv = rope_inv_freq(head_dim, theta, rope_scale)
    return pos.to(F32).unsqueeze(-1) * inv


def rotate_pairs(x: torch.Tensor, ang: torch.Tensor) -> torch.Tensor:
    """Rotate-half rotation of fp32 x [..., hd] by angles [..., hd/2]:
    y[d] = x[d] cos - x[d+h] sin; y[d+h] = x[d+h] cos + x[d] sin. cos/sin are taken in
    float64 of the fp32 angle, then rounded to fp32."""
    h = x.shape[-1] // 2
    a64 = ang.to(torch.float64)
    c, s = torch.cos(a64).to(F32), torch.sin(a64).to(F32)
    x0, x1 = x[..., :h], x[..., h:]
    return torch.cat([x0 * c - x1 * s, x1 * c + x0 * s], dim=-1)


def rope_llama(x: torch.Tensor, pos: torch.Tensor, theta: float, rope_scale: float = 1.0) -> torch.Tensor:
    """x [n, H, hd] (any float), pos [n] -> fp32 rotated."""
    ang = rope_angles(pos, x.shape[-1], theta, rope_scale)  # [n, hd/2]
    return rotate_pairs(x.to(F32), ang.unsqueeze(1))


def mrope_section_of(head_dim: int, sections) -> torch.Tensor:
    """Section index (0, 1, 2) of each rotation pair d < hd/2 from the cumulative sums of
    mrope_section (attention.cu:36-55: both halves of a pair use the section of d)."""
    cum = np.cumsum(sections)
    d = np.arange(head_dim // 2)
    return torch.from_numpy(np.where(d < cum[0], 0, np.where(d < cum[1], 1, 2)).astype(np.int64))


def mrope(x: torch.Tensor, position_ids: torch.Tensor, sections, theta: float, rope_scale: float = 1.0) -> torch.Tensor:
    """M-RoPE of x [S, H, hd] with position_ids [3, S]; returns bf16
    (mrope_kernel, attention.cu:17-72)."""
    hd = x.shape[-1]
    sec = mrope_section_of(hd, sections)                         # [hd/2]
    pos = position_ids.to(torch.int64)[sec, :].t()               # [S, hd/2]
    ang = pos.to(F32) * rope_inv_freq(hd, theta, rope_scale)     # [S, hd/2]
    return rotate_pairs(x.to(F32), ang.unsqueeze(1)).to(BF16)


# ---------------------------------------------------------------------------------
# Attention
# ---------------------------------------------------------------------------------
@dataclass
class AttnCtx:
    """Mirror of edge_fm::AttentionOpContext (src/operators/attention_op.h:20-39)."""
    num_qo_heads: int
    num_kv_heads: int
    head_dim: int
    rope_theta: float = 1.0e6
    rope_scale: float = 1.0
    rope: bool = True
    q_rope_pos_offset: int = 0
    k_rope_pos_offset: int = 0
    k_already_prerotated: bool = False


def attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, q_pos: torch.Tensor, ctx: AttnCtx,
              causal_offset: int | None) -> torch.Tensor:
    """General GQA attention. q [S, Hq, hd], k/v [L, Hkv, hd] (bf16), q_pos [S] the
    rotation positions of the queries. Query i sees keys j <= i + causal_offset when
    causal_offset is not None. Returns bf16 [S, Hq, hd]."""
    S, Hq, hd = q.shape
    L = k.shape[0]
    G = Hq // ctx.num_kv_heads
    qf = q.to(F32)
    kf = k.to(F32)
    if ctx.rope:
        qf = rope_llama(qf, q_pos, ctx.rope_theta, ctx.rope_scale)
        if not ctx.k_already_prerotated:
            kpos = torch.arange(L) + ctx.k_rope_pos_offset
            kf = rope_llama(kf, kpos, ctx.rope_theta, ctx.rope_scale)
    kf = kf.repeat_interleave(G, dim=1)            # [L, Hq, hd], head h -> kv head h // G
    vf = v.to(F32).repeat_interleave(G, dim=1)
    scores = torch.einsum("shd,lhd->hsl", qf, kf) / math.sqrt(hd)
    if causal_offset is not None:
        i = torch.arange(S).unsqueeze(1)
        j = torch.arange(L).unsqueeze(0)
        scores = scores.masked_fill((j > i + causal_offset).unsqueeze(0), float("-inf"))
    p = torch.softmax(scores, dim=-1)
    p = torch.nan_to_num(p, nan=0.0)
    o = torch.einsum("hsl,lhd->shd", p, vf)
    return o.to(BF16)


def attention_decode(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, kv_len: int, ctx: AttnCtx) -> torch.Tensor:
    """Decode: q [1, Hq, hd] attends keys [0, kv_len); q rotated at kv_len - 1 +
    q_rope_pos_offset, key j at j + k_rope_pos_offset (attention_op.cu:1428-1466,
    tests/operators/test_attention_decode.py:121-130)."""
    if kv_len == 0:
        return torch.zeros_like(q)
    qpos = torch.tensor([kv_len - 1 + ctx.q_rope_pos_offset])
    return attention(q, k[:kv_len], v[:kv_len], qpos, ctx, causal_offset=None)


def attention_prefill(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, ctx: AttnCtx, causal: bool = True) -> torch.Tensor:
    """Prefill: q [S, Hq, hd] over k/v [L, ...] with L >= S; query i has position
    i + q_rope_pos_offset and sees keys j <= i + (L - S) (attention_op.cu:1345-1426,
    qwen2_5.cpp:807-830)."""
    S = q.shape[0]
    L = k.shape[0]
    qpos = torch.arange(S) + ctx.q_rope_pos_offset
    return attention(q, k, v, qpos, ctx, causal_offset=(L - S) if causal else None)


def split_kv_merge(parts):
    """Log-sum-exp merge of split-KV partials [(o_unnormalised, m, l)] for one query
    row: the algebra used by split-KV decode (attention_op.cu:1212-1217, MergeStates)."""
    M = max(m for _, m, _ in parts)
    num = sum(math.exp(m - M) * o for o, m, _ in parts)
    den = sum(math.exp(m - M) * l for _, m, l in parts)
    return num / den


# ---------------------------------------------------------------------------------
# Embedding, sampler
# ---------------------------------------------------------------------------------
def embedding(ids: torch.Tensor, table: torch.Tensor, custom: torch.Tensor | None = None,
              embed_token_id: int = -1) -> torch.Tensor:
    """Row gather; ids in [embed_token_id, embed_token_id + len(custom)) read custom rows;
    ids outside the vocabulary give zero rows (embed_head.cu:63-132)."""
    V, H = table.shape
    out = torch.zeros(ids.numel(), H, dtype=table.dtype)
    for t, i in enumerate(ids.tolist()):
        if custom is not None and embed_token_id >= 0 and embed_token_id <= i < embed_token_id + custom.shape[0]:
            out[t] = custom[i - embed_token_id]
        elif 0 <= i < V:
            out[t] = table[i]
    return out


def argmax_lowest(logits: torch.Tensor) -> torch.Tensor:
    """Row-wise argmax with ties to the lowest index (sampler.cu:21-26)."""
    x = logits.to(torch.float64)
    m = x.max(dim=-1, keepdim=True).values
    idx = torch.arange(x.shape[-1]).expand_as(x)
    big = torch.full_like(idx, x.shape[-1])
    return torch.where(x == m, idx, big).min(dim=-1).values.to(torch.int32)


# ---------------------------------------------------------------------------------
# Qwen2.5 model
# ---------------------------------------------------------------------------------
@dataclass
class QwenConfig:
    hidden: int
    layers: int
    heads: int
    kv_heads: int
    head_dim: int
    inter: int
    vocab: int
    eps: float = 1e-6
    theta: float = 1.0e6
    tied: bool = True
    mrope_section: tuple | None = None  # (16, 24, 24) for Qwen2.5-VL

    @property
    def q_dim(self):
        return self.heads * self.head_dim

    @property
    def kv_dim(self):
        return self.kv_heads * self.head_dim


def fuse_weights(cfg: QwenConfig, w: dict) -> dict:
    """Fused layouts the reference builds at load: [Q;K;V] rows with [bq;bk;bv]
    (linear.cu:1629-1785), [up; gate] rows (linear.cu:1923-1943), tied LM head
    (linear.cu:2239-2286). Input: HF-style tensor names."""
    f = {"embed": w["model.embed_tokens.weight"], "final_norm": w["model.norm.weight"]}
    f["lm_head"] = w.get("lm_head.weight", w["model.embed_tokens.weight"]) if not cfg.tied else w["model.embed_tokens.weight"]
    for l in range(cfg.layers):
        p = f"model.layers.{l}."
        f[f"{l}.qkv_w"] = torch.cat([w[p + "self_attn.q_proj.weight"], w[p + "self_attn.k_proj.weight"],
                                      w[p + "self_attn.v_proj.weight"]], 0).contiguous()
        f[f"{l}.qkv_b"] = torch.cat([w[p + "self_attn.q_proj.bias"], w[p + "self_attn.k_proj.bias"],
                                      w[p + "self_attn.v_proj.bias"]], 0).contiguous()
        f[f"{l}.o_w"] = w[p + "self_attn.o_proj.weight"]
        f[f"{l}.gu_w"] = torch.cat([w[p + "mlp.up_proj.weight"], w[p + "mlp.gate_proj.weight"]], 0).contiguous()
        f[f"{l}.down_w"] = w[p + "mlp.down_proj.weight"]
        f[f"{l}.in_norm"] = w[p + "input_layernorm.weight"]
        f[f"{l}.post_norm"] = w[p + "post_attention_layernorm.weight"]
    return f


def random_weights(cfg: QwenConfig, seed: int, std: float = 0.02) -> dict:
    """Seeded N(0, std) bf16 weights under HF Qwen2 tensor names (norm weights N(1, std)
    so RMSNorm is not degenerate). Deterministic for a given seed."""
    g = torch.Generator().manual_seed(seed)

    def n(*shape, mean=0.0):
        return (torch.randn(*shape, generator=g) * std + mean).to(BF16)

    w = {"model.embed_tokens.weight": n(cfg.vocab, cfg.hidden), "model.norm.weight": n(cfg.hidden, mean=1.0)}
    for l in range(cfg.layers):
        p = f"model.layers.{l}."
        w[p + "self_attn.q_proj.weight"] = n(cfg.q_dim, cfg.hidden)
        w[p + "self_attn.k_proj.weight"] = n(cfg.kv_dim, cfg.hidden)
        w[p + "self_attn.v_proj.weight"] = n(cfg.kv_dim, cfg.hidden)
        w[p + "self_attn.q_proj.bias"] = n(cfg.q_dim)
        w[p + "self_attn.k_proj.bias"] = n(cfg.kv_dim)
        w[p + "self_attn.v_proj.bias"] = n(cfg.kv_dim)
        w[p + "self_attn.o_proj.weight"] = n(cfg.hidden, cfg.q_dim)
        w[p + "mlp.gate_proj.weight"] = n(cfg.inter, cfg.hidden)
        w[p + "mlp.up_proj.weight"] = n(cfg.inter, cfg.hidden)
        w[p + "mlp.down_proj.weight"] = n(cfg.hidden, cfg.inter)
        w[p + "input_layernorm.weight"] = n(cfg.hidden, mean=1.0)
        w[p + "post_attention_layernorm.weight"] = n(cfg.hidden, mean=1.0)
    if not cfg.tied:
        w["lm_head.weight"] = n(cfg.vocab, cfg.hidden)
    return w


@dataclass
class QwenState:
    """Per-request KV cache (un-rotated K for text models, M-RoPE-rotated K for VL) and
    the number of valid rows."""
    k: list = field(default_factory=list)
    v: list = field(default_factory=list)
    length: int = 0


class Qwen2Oracle:
    """Qwen2_5::forward_impl (qwen2_5.cpp:534-930) on the CPU with Appendix-A rounding."""

    def __init__(self, cfg: QwenConfig, fused: dict, max_tokens: int, cache_f32: bool = False):
        """cache_f32 keeps an fp32 copy of every weight matrix so repeated steps do not
        re-convert bf16 -> fp32 (same values, faster on large models)."""
        self.cfg = cfg
        self.w = {k: v.to(F32) for k, v in fused.items()} if cache_f32 else fused
        self.max_tokens = max_tokens

    def new_state(self) -> QwenState:
        c = self.cfg
        st = QwenState()
        st.k = [torch.zeros(self.max_tokens, c.kv_heads, c.head_dim, dtype=BF16) for _ in range(c.layers)]
        st.v = [torch.zeros(self.max_tokens, c.kv_heads, c.head_dim, dtype=BF16) for _ in range(c.layers)]
        return st

    def _layers(self, st: QwenState, h: torch.Tensor, position_ids: torch.Tensor | None) -> torch.Tensor:
        """h [S, H] bf16 embeddings of S new tokens at cache rows [st.length, +S).
        Returns the final hidden state after the last fused add + RMSNorm [S, H]."""
        c, w = self.cfg, self.w
        S = h.shape[0]
        base = st.length
        L = base + S
        actx = AttnCtx(c.heads, c.kv_heads, c.head_dim, rope_theta=c.theta, rope=c.mrope_section is None,
                       q_rope_pos_offset=base)
        residual = None
        x = h
        for l in range(c.layers):
            if l == 0:
                n = rms_norm(x, w[f"{l}.in_norm"], c.eps)
                residual = x
            else:
                n, residual = fused_add_rms_norm(x, residual, w[f"{l}.in_norm"], c.eps)
            qkv = linear(n, w[f"{l}.qkv_w"], w[f"{l}.qkv_b"])
            q = qkv[:, : c.q_dim].reshape(S, c.heads, c.head_dim)
            k = qkv[:, c.q_dim: c.q_dim + c.kv_dim].reshape(S, c.kv_heads, c.head_dim)
            v = qkv[:, c.q_dim + c.kv_dim:].reshape(S, c.kv_heads, c.head_dim)
            if c.mrope_section is not None:
                q = mrope(q, position_ids, c.mrope_section, c.theta)
                k = mrope(k, position_ids, c.mrope_section, c.theta)
            st.k[l][base:L] = k
            st.v[l][base:L] = v
            o = attention_prefill(q, st.k[l][:L], st.v[l][:L], actx, causal=True)
            a = linear(o.reshape(S, c.q_dim), w[f"{l}.o_w"])
            n2, residual = fused_add_rms_norm(a, residual, w[f"{l}.post_norm"], c.eps)
            m = gate_up_swiglu(n2, w[f"{l}.gu_w"])
            x = linear(m, w[f"{l}.down_w"])
        out, _ = fused_add_rms_norm(x, residual, w["final_norm"], c.eps)
        st.length = L
        return out

    def forward(self, st: QwenState, ids: torch.Tensor, embeds: torch.Tensor | None = None,
                position_ids: torch.Tensor | None = None) -> torch.Tensor:
        """Run S new tokens (prefill when S > 1, a decode step when S == 1); return the
        fp32 logits of the last row (qwen2_5.cpp:891-929)."""
        h = embeds if embeds is not None else embedding(ids, self.w["embed"])
        x = self._layers(st, h, position_ids)
        return linear(x[-1:], self.w["lm_head"], out_f32=True)[0]

    def generate_greedy(self, prompt: torch.Tensor, max_new_tokens: int, forced: list | None = None):
        """Greedy loop: prefill -> sample, then one decode step per token
        (standard_engine.cpp:872-1094). Token count capped by
        min(max_new_tokens, max_tokens - len(prompt) + 1) (scheduler.cpp:123-134).
        If `forced` is given the next input token is forced[i] (teacher forcing) and
        the returned list holds (argmax, top1 - top2 margin) per step."""
        st = self.new_state()
        n = min(max_new_tokens, self.max_tokens - prompt.numel() + 1)
        logits = self.forward(st, prompt)
        out = []
        for i in range(n):
            tok = int(argmax_lowest(logits.unsqueeze(0))[0])
            top2 = torch.topk(logits.to(torch.float64), 2).values
            out.append((tok, float(top2[0] - top2[1])))
            if i + 1 == n:
                break
            nxt = forced[i] if forced is not None else tok
            logits = self.forward(st, torch.tensor([nxt], dtype=torch.int32))
        return out


# ---------------------------------------------------------------------------------
# SageAttention-style int8 QK^T prefill attention. The reference
# has no implementation (README.md:23 only names it), so this restates the published
# method (Zhang et al., "SageAttention: Accurate 8-Bit Attention for Plug-and-play
# Inference Acceleration", 2024) with the choices fixed here:
#   * K smoothing: K_s = K - mean_over_tokens(K) per (KV head, channel); the mean is
#     accumulated in float64 and rounded once to fp32. Softmax is invariant to it.
#   * symmetric int8 per (128-token block, head) for Q and for K_s:
#     scale = max|x| / 127 (fp32; 1.0 for an all-zero block), x8 = round-half-even(x /
#     scale) clamped to [-127, 127].
#   * S = int32(Q8 . K8^T); score_log2 = float(S) * ((sq * sk) * (log2(e) / sqrt(hd)))
#     in fp32, in that order.
#   * causal online softmax in fp32 (base 2), P rounded to bf16, O = P . V with fp32
#     accumulation, normalised, rounded to bf16.
# The integer part (Q8, K8, scales, S) is bit-exact by construction and is compared
# exactly; the output is compared with the bf16 attention within tolerance.
# ---------------------------------------------------------------------------------
SAGE_BLOCK = 128


def sage_kmean(k: torch.Tensor) -> torch.Tensor:
    """Per (KV head, channel) mean over tokens: float64 sum / L, rounded to fp32. k [L, Hkv, hd]."""
    return (k.to(torch.float64).sum(0) / k.shape[0]).to(F32)


def sage_quant_blocks(x: torch.Tensor, block: int = SAGE_BLOCK):
    """Symmetric int8 per (block of tokens, head). x fp32 [T, H, hd] -> (int8 [T, H, hd],
    scales fp32 [ceil(T/block), H])."""
    T, H, hd = x.shape
    nb = (T + block - 1) // block
    q8 = torch.empty(T, H, hd, dtype=torch.int8)
    scales = torch.empty(nb, H, dtype=F32)
    for b in range(nb):
        xb = x[b * block:(b + 1) * block]                       # [t, H, hd]
        amax = xb.abs().amax(dim=(0, 2))                        # [H] fp32
        sc = torch.where(amax > 0, amax / torch.tensor(127.0, dtype=F32), torch.ones_like(amax))
        scales[b] = sc
        q8[b * block:(b + 1) * block] = torch.clamp(torch.round(xb / sc[None, :, None]), -127, 127).to(torch.int8)
    return q8, scales


def sage_quantize(q: torch.Tensor, k: torch.Tensor, block: int = SAGE_BLOCK):
    """(q8, sq, k8, sk, kmean) for q [S, Hq, hd], k [L, Hkv, hd] (bf16)."""
    kmean = sage_kmean(k)
    ks = k.to(F32) - kmean[None]
    q8, sq = sage_quant_blocks(q.to(F32), block)
    k8, sk = sage_quant_blocks(ks, block)
    return q8, sq, k8, sk, kmean


def sage_scores_int32(q8: torch.Tensor, k8: torch.Tensor, num_kv_heads: int) -> torch.Tensor:
    """Exact int32 Q8 . K8^T per query head: [Hq, S, L] (int64 matmul, no overflow)."""
    G = q8.shape[1] // num_kv_heads
    kk = k8.to(torch.int64).repeat_interleave(G, dim=1)          # [L, Hq, hd]
    return torch.einsum("shd,lhd->hsl", q8.to(torch.int64), kk).to(torch.int32)


def sage_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, num_kv_heads: int, causal: bool = True,
                   block: int = SAGE_BLOCK) -> torch.Tensor:
    """SageAttention-style prefill attention, q [S, Hq, hd], k/v [L, Hkv, hd] bf16 -> bf16
    [S, Hq, hd]. Query i sees keys j <= i + (L - S) when causal."""
    S, Hq, hd = q.shape
    L = k.shape[0]
    G = Hq // num_kv_heads
    q8, sq, k8, sk, _ = sage_quantize(q, k, block)
    acc = sage_scores_int32(q8, k8, num_kv_heads).to(F32)        # [Hq, S, L]
    scale_log2 = torch.tensor(1.4426950408889634 / math.sqrt(hd), dtype=F32)
    sq_row = sq.repeat_interleave(block, 0)[:S].t()               # [Hq, S]
    sk_col = sk.repeat_interleave(block, 0)[:L].t().repeat_interleave(G, 0)  # [Hq, L]
    coef = (sq_row[:, :, None] * sk_col[:, None, :]) * scale_log2
    s2 = acc * coef                                              # base-2 scores
    if causal:
        i = torch.arange(S).unsqueeze(1)
        j = torch.arange(L).unsqueeze(0)
        s2 = s2.masked_fill((j > i + (L - S)).unsqueeze(0), float("-inf"))
    m = s2.amax(-1, keepdim=True)
    p = torch.exp2(s2 - m)
    den = p.sum(-1, keepdim=True)
    pb = p.to(BF16).to(F32)                                      # P rounded to bf16 for PV
    vf = v.to(F32).repeat_interleave(G, dim=1)                    # [L, Hq, hd]
    o = torch.einsum("hsl,lhd->shd", pb, vf) / den.permute(1, 0, 2)
    return o.to(BF16)


# ---------------------------------------------------------------------------------
# Temperature / top-p sampling. The reference samples with
# FlashInfer OnlineSoftmax + SamplingFromProb(seed, offset 0) and has no top-p
# (src/layers/sampler.cu:251-298); its RNG is cuRAND inside un-vendored FlashInfer, so
# index parity with it is unpinned. This build defines the sampler exactly, with all
# mass arithmetic in integers so that it is reproducible bit for bit:
#   m      = max_i l_i                                   (fp32 logits)
#   e_i    = expf((l_i - m) / T)                         (fp32 subtract, divide, exp)
#   w_i    = rint(e_i * 2^44)                            (uint64; sum fits for V <= 2^20)
#   W      = sum_i w_i
#   nucleus: all i when top_p >= 1, else { i : e_i >= tau } with tau the largest fp32
#            value such that sum_{e_j >= tau} w_j >= ceil(top_p * W) (top_p as float64)
#   x      = philox4x32_10(counter = (off_lo, off_hi, 0, 0), key = (seed_lo, seed_hi))[0]
#   r      = floor(N * (x >> 8) / 2^24), N = nucleus mass  (0 <= r < N)
#   token  = the smallest nucleus index i with sum_{j <= i, j in nucleus} w_j > r
# offset = the index of the token in the response, so every step draws a fresh number.
# Philox4x32-10 is pinned by its published known-answer vectors.
# ---------------------------------------------------------------------------------
_PHILOX_M0, _PHILOX_M1 = 0xD2511F53, 0xCD9E8D57
_PHILOX_W0, _PHILOX_W1 = 0x9E3779B9, 0xBB67AE85
SAMPLE_MASS_BITS = 44


def philox4x32_10(counter, key):
    """Philox4x32 with 10 rounds (Salmon, Moraes, Dror, Shaw, SC'11). counter: 4 uint32,
    key: 2 uint32 -> 4 uint32."""
    c = [int(x) & 0xFFFFFFFF for x in counter]
    k0, k1 = int(key[0]) & 0xFFFFFFFF, int(key[1]) & 0xFFFFFFFF
    for r in range(10):
        p0 = _PHILOX_M0 * c[0]
        p1 = _PHILOX_M1 * c[2]
        hi0, lo0 = p0 >> 32, p0 & 0xFFFFFFFF
        hi1, lo1 = p1 >> 32, p1 & 0xFFFFFFFF
        c = [hi1 ^ c[1] ^ k0, lo1, hi0 ^ c[3] ^ k1, lo0]
        if r < 9:
            k0 = (k0 + _PHILOX_W0) & 0xFFFFFFFF
            k1 = (k1 + _PHILOX_W1) & 0xFFFFFFFF
    return c


def sampling_bits(seed: int, offset: int) -> int:
    """The 24 random bits one sampling call consumes."""
    x = philox4x32_10((offset & 0xFFFFFFFF, (offset >> 32) & 0xFFFFFFFF, 0, 0),
                      (seed & 0xFFFFFFFF, (seed >> 32) & 0xFFFFFFFF))[0]
    return x >> 8


def sample_masses(logits, temperature: float):
    """fp32 e_i and uint64 w_i of one logits row (numpy float32 arithmetic)."""
    l = np.asarray(logits, dtype=np.float32)
    x = (l - l.max()) / np.float32(temperature)
    e = np.exp(x.astype(np.float32)).astype(np.float32)
    w = np.rint(e.astype(np.float64) * float(2 ** SAMPLE_MASS_BITS)).astype(np.uint64)
    return e, w


def nucleus_threshold(e, w, top_p: float):
    """Smallest kept e (tau) of the top-p nucleus; brute force over the distinct values."""
    total = int(w.sum(dtype=np.uint64))
    need = math.ceil(float(top_p) * total)
    order = np.argsort(-e, kind="stable")
    vals = e[order]
    cum = np.cumsum(w[order], dtype=np.uint64)
    # first position whose cumulative mass reaches `need`, then widen to all ties
    pos = int(np.searchsorted(cum, np.uint64(need), side="left"))
    pos = min(pos, len(vals) - 1)
    return np.float32(vals[pos])


def sample_top_p(logits, temperature: float, top_p: float, seed: int, offset: int):
    """Returns (token, info) for one fp32 logits row. info: nucleus size, tau, masses and
    the relative distance of the random target to the nearest CDF boundary."""
    top_p = float(np.float32(top_p))
    e, w = sample_masses(logits, temperature)
    if top_p >= 1.0:
        keep = np.ones(e.shape, dtype=bool)
        tau = np.float32(0.0)
    else:
        tau = nucleus_threshold(e, w, top_p)
        keep = e >= tau
    wk = np.where(keep, w, np.uint64(0))
    n_mass = int(wk.sum(dtype=np.uint64))
    bits = sampling_bits(seed, offset)
    r = (n_mass * bits) >> 24
    cdf = np.cumsum(wk, dtype=np.uint64)
    token = int(np.searchsorted(cdf, np.uint64(r), side="right"))
    return token, {"nucleus": int(keep.sum()), "tau": float(tau), "total": int(w.sum(dtype=np.uint64)),
                   "mass": n_mass, "r": r}


def sample_margin(logits, temperature: float, top_p: float, seed: int, offset: int) -> float:
    """Smallest relative distance of a sampling decision to its boundary: the random
    target r to any CDF step (/ N) and ceil(top_p * W) to any cumulative sorted mass
    (/ W). Below ~1e-6 a one-ulp difference in some e_i may change the token."""
    top_p = float(np.float32(top_p))
    e, w = sample_masses(logits, temperature)
    total = int(w.sum(dtype=np.uint64))
    margin = 1.0
    keep = np.ones(e.shape, dtype=bool)
    if top_p < 1.0:
        need = math.ceil(float(top_p) * total)
        cum = np.cumsum(w[np.argsort(-e, kind="stable")], dtype=np.uint64).astype(np.float64)
        margin = min(margin, float(np.min(np.abs(cum - need))) / total)
        keep = e >= nucleus_threshold(e, w, top_p)
    wk = np.where(keep, w, np.uint64(0))
    n_mass = int(wk.sum(dtype=np.uint64))
    r = (n_mass * sampling_bits(seed, offset)) >> 24
    cdf = np.cumsum(wk, dtype=np.uint64).astype(np.float64)
    return min(margin, float(np.min(np.abs(cdf - r))) / max(n_mass, 1))
