"""Host-side helpers to stand up an EdgeFM engine on MI355X from Python.

* write an HF-style ``config.json`` for a Qwen2.5 / Qwen2.5-VL shape,
* write the engine JSON (merged by the runtime over configs/engine_default.json),
* register device-resident weight tensors with the runtime's WeightLoader so no
  safetensors file has to be written (zero-copy views; the caller keeps the torch
  tensors alive for the engine's lifetime),
* seeded synthetic weights generated directly on the GPU.

Requires the built ``edge_fm`` module next to this file.
"""
from __future__ import annotations

import json
import os
from dataclasses import dataclass

import edge_fm  # noqa: F401  (fails loudly when the module is not built)


@dataclass
class ModelShape:
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
    mrope_section: tuple | None = None

    @property
    def q_dim(self):
        return self.heads * self.head_dim

    @property
    def kv_dim(self):
        return self.kv_heads * self.head_dim


# BASELINE shapes
QWEN25_0P5B = ModelShape(896, 24, 14, 2, 64, 4864, 151936)
QWEN25_1P5B = ModelShape(1536, 28, 12, 2, 128, 8960, 151936)
QWEN25_VL_3B = ModelShape(2048, 36, 16, 2, 128, 11008, 151936, mrope_section=(16, 24, 24))
QWEN25_7B = ModelShape(3584, 28, 28, 4, 128, 18944, 152064, tied=False)


def write_model_dir(path: str, shape: ModelShape, eos_token_id=None) -> str:
    os.makedirs(path, exist_ok=True)
    cfg = {
        "model_type": "qwen2_5_vl" if shape.mrope_section else "qwen2",
        "hidden_size": shape.hidden,
        "intermediate_size": shape.inter,
        "num_hidden_layers": shape.layers,
        "num_attention_heads": shape.heads,
        "num_key_value_heads": shape.kv_heads,
        "head_dim": shape.head_dim,
        "vocab_size": shape.vocab,
        "rms_norm_eps": shape.eps,
        "rope_theta": shape.theta,
        "tie_word_embeddings": shape.tied,
        "torch_dtype": "bfloat16",
    }
    if shape.mrope_section:
        cfg["rope_scaling"] = {"type": "mrope", "mrope_section": list(shape.mrope_section)}
    if eos_token_id is not None:
        cfg["eos_token_id"] = eos_token_id
    with open(os.path.join(path, "config.json"), "w") as f:
        json.dump(cfg, f)
    return path


def write_checkpoint(model_dir: str, weights: dict, shards: int = 1, rename=None, extra: dict | None = None) -> list:
    """Write HF-named tensors as a safetensors checkpoint under model_dir: one
    model.safetensors (shards == 1) or model-0000i-of-0000n.safetensors shards (tensors
    dealt round-robin in name order). rename maps a tensor name to the name stored (a
    Qwen2.5-VL checkpoint prefixes the language model: model.language_model.*); extra
    tensors are stored as given (e.g. a vision tower the text model ignores). Returns the
    file paths."""
    from safetensors.torch import save_file

    os.makedirs(model_dir, exist_ok=True)
    named = {(rename(k) if rename else k): v.detach().cpu().contiguous() for k, v in weights.items()}
    named.update({k: v.detach().cpu().contiguous() for k, v in (extra or {}).items()})
    names = sorted(named)
    if shards == 1:
        paths = [os.path.join(model_dir, "model.safetensors")]
        save_file(named, paths[0])
        return paths
    paths = []
    for i in range(shards):
        part = {k: named[k] for k in names[i::shards]}
        path = os.path.join(model_dir, f"model-{i + 1:05d}-of-{shards:05d}.safetensors")
        save_file(part, path)
        paths.append(path)
    return paths


def write_compact_vocab_mapping(path: str, original_vocab_size: int, new_to_old, special_token_ids,
                                fmt: str = "edgefm.compact_vocab.v1") -> str:
    """Write an ``edgefm.compact_vocab.v1`` mapping: compact id n is original id new_to_old[n];
    every other original id maps to -1."""
    old_to_new = [-1] * original_vocab_size
    for n, o in enumerate(new_to_old):
        old_to_new[o] = n
    with open(path, "w") as f:
        json.dump({"format": fmt, "original_vocab_size": original_vocab_size,
                   "compact_vocab_size": len(new_to_old), "old_to_new": old_to_new,
                   "new_to_old": list(new_to_old), "special_token_ids": list(special_token_ids)}, f)
    return path


def write_engine_config(path: str, model_dir: str, *, max_tokens: int = 4096, max_new_tokens: int = 256,
                        prefix_token_ids=None, use_graph: bool = True, temperature: float = 0.0,
                        top_p: float = 1.0, seed: int = 0, lm_head_top1: bool = True, model_name: str = "",
                        operator_impl_table_path: str = "", extra_slots=None,
                        stop_token_ids=None, compact_vocab=None, decode_fused_qkv_attention=None,
                        debug_logits: bool = False) -> str:
    slots = [{"request_id": 0, "prefix_token_ids": list(prefix_token_ids or []), "max_tokens": max_tokens}]
    for s in extra_slots or []:
        slots.append(s)
    cfg = {
        "model_name": model_name,
        "runtime": {"device": "gpu", "device_id": 0, "use_cuda_graph": use_graph, "lm_head_top1": lm_head_top1},
        "prefill_model_path": model_dir,
        "operator_impl_table_path": operator_impl_table_path,
        "kvcache": {"dtype": "bf16", "requests": slots},
        "sampling": {"max_new_tokens": max_new_tokens, "temperature": temperature, "top_p": top_p, "seed": seed,
                     "stop_token_ids": list(stop_token_ids or [])},
    }
    if decode_fused_qkv_attention is not None:
        cfg["runtime"]["decode_fused_qkv_attention"] = bool(decode_fused_qkv_attention)
    if compact_vocab is not None:
        cfg["compact_vocab"] = compact_vocab
    if debug_logits:
        cfg["runtime"]["debug_logits"] = True
    with open(path, "w") as f:
        json.dump(cfg, f)
    return path


def register_weights(weights: dict) -> dict:
    """Register HF-named device tensors (bf16, contiguous, on cuda) with the runtime's
    WeightLoader for the prefill stage. Returns the dict, which must stay referenced
    while the engine exists."""
    import torch

    loader = edge_fm.WeightLoader.instance()
    loader.clear_stage(edge_fm.ModelStage.Prefill)
    for name, t in weights.items():
        if not (t.is_cuda and t.is_contiguous() and t.dtype == torch.bfloat16):
            raise ValueError(f"weight {name} must be a contiguous bf16 cuda tensor")
        loader.register_tensor(edge_fm.ModelStage.Prefill, name,
                               edge_fm.Tensor(t.data_ptr(), list(t.shape), edge_fm.DType.BFloat16,
                                              edge_fm.Device.GPU, t.device.index or 0, False))
    return weights


def synthetic_weights_gpu(shape: ModelShape, seed: int, std: float = 0.02, device: str = "cuda:0") -> dict:
    """Seeded N(0, std) bf16 weights for every tensor of the architecture, generated on
    the GPU (RMSNorm weights are ones, their usual initialisation)."""
    import torch

    g = torch.Generator(device=device).manual_seed(seed)

    def n(*s):
        t = torch.empty(*s, dtype=torch.bfloat16, device=device)
        t.normal_(0.0, std, generator=g)
        return t

    def ones(*s):
        return torch.ones(*s, dtype=torch.bfloat16, device=device)

    w = {"model.embed_tokens.weight": n(shape.vocab, shape.hidden), "model.norm.weight": ones(shape.hidden)}
    for layer in range(shape.layers):
        p = f"model.layers.{layer}."
        w[p + "self_attn.q_proj.weight"] = n(shape.q_dim, shape.hidden)
        w[p + "self_attn.k_proj.weight"] = n(shape.kv_dim, shape.hidden)
        w[p + "self_attn.v_proj.weight"] = n(shape.kv_dim, shape.hidden)
        w[p + "self_attn.q_proj.bias"] = n(shape.q_dim)
        w[p + "self_attn.k_proj.bias"] = n(shape.kv_dim)
        w[p + "self_attn.v_proj.bias"] = n(shape.kv_dim)
        w[p + "self_attn.o_proj.weight"] = n(shape.hidden, shape.q_dim)
        w[p + "mlp.gate_proj.weight"] = n(shape.inter, shape.hidden)
        w[p + "mlp.up_proj.weight"] = n(shape.inter, shape.hidden)
        w[p + "mlp.down_proj.weight"] = n(shape.hidden, shape.inter)
        w[p + "input_layernorm.weight"] = ones(shape.hidden)
        w[p + "post_attention_layernorm.weight"] = ones(shape.hidden)
    if not shape.tied:
        w["lm_head.weight"] = n(shape.vocab, shape.hidden)
    return w
