"""The layer tier's Python surface matches the reference's per-layer bindings
(src/python/pybind_debug.cpp:486-1580): class names, constructor and method argument
names in order, and defaults. Host only: nothing is constructed on a device."""
import re

import pytest

import edge_fm

# (class, method) -> argument names after self, as bound by the reference
SURFACE = {
    ("AttentionLayer", "__init__"): ["config_path"],
    ("AttentionLayer", "forward_prefill"): ["q", "k", "v", "o", "causal", "stream", "q_stride_n", "q_stride_h",
                                            "kv_stride_n", "kv_stride_h", "k_stride_n", "k_stride_h"],
    ("AttentionLayer", "forward_decode"): ["q", "k", "v", "o", "stream", "max_kv_len", "d_kv_len"],
    ("RMSNormLayer", "__init__"): ["layer_id", "config_path", "weight_type"],
    ("RMSNormLayer", "forward_rmsnorm"): ["input", "output", "stream"],
    ("RMSNormLayer", "forward_fused_add_rmsnorm"): ["inout", "residual", "stream"],
    ("ActivationLayer", "__init__"): ["config_path"],
    ("ActivationLayer", "forward_silu_and_mul"): ["input", "output", "stream", "stage"],
    ("ActivationLayer", "forward_silu_and_mul_up_gate"): ["input", "output", "stream", "stage"],
    ("SamplerLayer", "__init__"): ["config_path"],
    ("SamplerLayer", "forward"): ["logits", "token_ids", "stream"],
    ("LinearLayer", "__init__"): ["layer_prefix", "config_path", "in_features", "out_features"],
    ("LinearLayer", "forward_fp16_bf16"): ["input", "output", "stream", "stage"],
    ("LinearLayer", "debug_cached_impl_info"): ["stage", "m"],
    ("LinearLayer", "debug_weight_tensor_info"): ["stage"],
    ("FusedQKVLinearLayer", "__init__"): ["layer_prefix_base", "config_path", "in_features", "q_out_features",
                                          "k_out_features", "v_out_features"],
    ("FusedGateUpLinearLayer", "__init__"): ["layer_prefix_base", "config_path", "in_features", "gate_out_features",
                                             "up_out_features"],
    ("FusedGateUpLinearLayer", "try_forward_decode_swiglu_fused"): ["input", "output", "stream"],
    ("FusedGateUpLinearLayer", "try_forward_prefill_swiglu_fused"): ["input", "output", "stream"],
    ("LMHeadLinearLayer", "__init__"): ["config_path", "in_features", "out_features", "layer_prefix"],
    ("LMHeadLinearLayer", "try_forward_top1"): ["input", "token_out", "stream", "stage"],
    ("EmbedHeadLayer", "__init__"): ["config_path"],
    ("EmbedHeadLayer", "forward_for_tokens"): ["token_ids", "output", "stream"],
    ("EmbedHeadLayer", "forward_for_embeddings"): ["token_ids", "embeddings", "output", "embed_token_id", "stream"],
    ("KVManager", "__init__"): ["config_path"],
    ("KVManager", "get_read_kvcache"): ["request_id"],
    ("KVManager", "get_write_kvcache"): ["request_id"],
    ("KVManager", "is_request_valid"): ["request_id"],
    ("Tensor", "from_dlpack"): ["capsule"],
}

DEFAULTS = {
    ("AttentionLayer", "forward_prefill"): {"causal": "True", "stream": "0"},
    ("AttentionLayer", "forward_decode"): {"stream": "0", "max_kv_len": "0", "d_kv_len": "None"},
    ("RMSNormLayer", "__init__"): {"weight_type": "'input'"},
    ("ActivationLayer", "forward_silu_and_mul"): {"stage": "'Prefill'"},
    ("LinearLayer", "debug_cached_impl_info"): {"stage": "'Decode'", "m": "1"},
    ("LMHeadLinearLayer", "__init__"): {"layer_prefix": "'lm_head'"},
    ("LMHeadLinearLayer", "try_forward_top1"): {"stage": "'Decode'"},
    ("EmbedHeadLayer", "forward_for_embeddings"): {"embed_token_id": "-1"},
}


def _args(doc: str, name: str):
    """Argument names and defaults of the first pybind11 signature line of `name`."""
    line = next(l for l in doc.splitlines() if l.startswith(name + "(") or re.match(r"^\d+\. " + name, l) or
                l.startswith("__init__(") or l.startswith("from_dlpack("))
    inner = line[line.index("(") + 1: line.rindex(")")]
    out = {}
    for part in re.split(r", (?=[a-z_]+:)", inner):
        if ":" not in part:
            continue
        n, rest = part.split(":", 1)
        n = n.strip()
        if n == "self":
            continue
        out[n] = rest.split("=", 1)[1].strip() if "=" in rest else None
    return out


@pytest.mark.parametrize("cls,method", sorted(SURFACE))
def test_binding_matches_reference_signature(cls, method):
    fn = getattr(getattr(edge_fm, cls), method)
    args = _args(fn.__doc__, method)
    assert list(args) == SURFACE[(cls, method)]
    for k, v in DEFAULTS.get((cls, method), {}).items():
        assert args[k] == v, f"{cls}.{method} default of {k}: {args[k]} != {v}"


def test_fused_layers_derive_from_linear_layer():
    for name in ("FusedQKVLinearLayer", "FusedGateUpLinearLayer", "LMHeadLinearLayer"):
        assert issubclass(getattr(edge_fm, name), edge_fm.LinearLayer)
    assert hasattr(edge_fm, "KVSlotStatus") and hasattr(edge_fm, "KVManagerStatus")
