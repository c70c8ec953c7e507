"""ctypes binding of the edgefm_hip C ABI (include/edgefm_hip.h).

This is the stub a maintainer of the reference would add to reach the HIP kernels
from Python without the pybind module: every entry point of the header is declared
here with its exact C signature. Pointers are passed as integers (e.g. a torch
tensor's data_ptr()), the stream as the raw hipStream_t handle.

Loading fails loudly when the library has not been built: there is no fallback.
"""
from __future__ import annotations

import ctypes
import os
from ctypes import POINTER, c_char_p, c_float, c_int32, c_int64, c_size_t, c_uint32, c_uint64, c_void_p

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libedgefm_hip.so")

EFM_OK = 0
EFM_ERR_INVALID_ARGUMENT = 1
EFM_ERR_UNSUPPORTED = 2
EFM_ERR_DEVICE = 3
EFM_ERR_WORKSPACE = 4

EFM_DTYPE_F32 = 0
EFM_DTYPE_F16 = 1
EFM_DTYPE_BF16 = 2
EFM_DTYPE_I32 = 3

EFM_POS_NONE = 0
EFM_POS_ROPE_LLAMA = 1
EFM_K_PREROTATED_EXCEPT_NEWEST = 2

EFM_LAYOUT_GATE_UP = 0
EFM_LAYOUT_UP_GATE = 1

EFM_ATTENTION_DECODE_NOALLOC_SCRATCH_BYTES = 2359296

EFM_KNOB_DECODE_REGISTER = 0
EFM_KNOB_PREFILL_REGISTER = 1
EFM_KNOB_PREFILL_SHAPE = 2
EFM_KNOB_GEMM_TILE = 3
EFM_KNOB_FRONT_WAIT_TIMEOUT = 4
EFM_KNOB_DECODE_TILE = 5


class AttentionCtx(ctypes.Structure):
    """efm_attention_ctx (mirror of edge_fm::AttentionOpContext)."""
    _fields_ = [
        ("num_qo_heads", c_uint32),
        ("num_kv_heads", c_uint32),
        ("head_dim", c_uint32),
        ("q_stride_n", c_uint32),
        ("q_stride_h", c_uint32),
        ("k_stride_n", c_uint32),
        ("k_stride_h", c_uint32),
        ("kv_stride_n", c_uint32),
        ("kv_stride_h", c_uint32),
        ("rope_scale", c_float),
        ("rope_theta", c_float),
        ("q_rope_pos_offset", c_uint32),
        ("k_rope_pos_offset", c_uint32),
        ("dtype", c_int32),
        ("pos_encoding", c_int32),
        ("k_already_prerotated", c_int32),
    ]


def make_attention_ctx(num_qo_heads, num_kv_heads, head_dim, *, rope=True, rope_theta=1.0e6, rope_scale=1.0,
                       q_rope_pos_offset=0, k_rope_pos_offset=0, k_already_prerotated=False, q_stride_n=0,
                       q_stride_h=0, k_stride_n=0, k_stride_h=0, kv_stride_n=0, kv_stride_h=0) -> AttentionCtx:
    return AttentionCtx(num_qo_heads, num_kv_heads, head_dim, q_stride_n, q_stride_h, k_stride_n, k_stride_h,
                        kv_stride_n, kv_stride_h, rope_scale, rope_theta, q_rope_pos_offset, k_rope_pos_offset,
                        EFM_DTYPE_BF16, EFM_POS_ROPE_LLAMA if rope else EFM_POS_NONE, int(k_already_prerotated))


# name -> (restype, argtypes)
SIGNATURES = {
    "efm_last_error": (c_char_p, []),
    "efm_version": (c_char_p, []),
    "efm_init": (c_int32, []),
    "efm_attention_decode_workspace_bytes": (c_size_t, [POINTER(AttentionCtx), c_uint32]),
    "efm_attention_decode_noalloc": (c_int32, [POINTER(AttentionCtx), c_void_p, c_void_p, c_void_p, c_void_p, c_uint32,
                                               c_void_p, c_uint32, c_void_p]),
    "efm_attention_decode": (c_int32, [POINTER(AttentionCtx), c_void_p, c_void_p, c_void_p, c_void_p, c_uint32,
                                       c_void_p, c_uint32, c_void_p, c_size_t, c_void_p]),
    "efm_decode_attention_partials": (c_int32, [POINTER(AttentionCtx), c_void_p, c_void_p, c_void_p, c_void_p,
                                                c_uint32, c_void_p, c_size_t, c_void_p]),
    "efm_decode_attention_merge_o_proj": (c_int32, [POINTER(AttentionCtx), c_void_p, c_uint32, c_void_p, c_size_t,
                                                    c_void_p, c_int32, c_void_p, c_void_p]),
    "efm_decode_attention_merge_o_proj_supported": (c_int32, [POINTER(AttentionCtx), c_uint32]),
    "efm_attention_prefill": (c_int32, [POINTER(AttentionCtx), c_void_p, c_void_p, c_void_p, c_void_p, c_uint32,
                                        c_uint32, c_int32, c_void_p]),
    "efm_attention_prefill_sage_int8_workspace_bytes": (c_size_t, [POINTER(AttentionCtx), c_uint32, c_uint32]),
    "efm_attention_prefill_sage_int8": (c_int32, [POINTER(AttentionCtx), c_void_p, c_void_p, c_void_p, c_void_p,
                                                  c_uint32, c_uint32, c_int32, c_void_p, c_size_t, c_void_p]),
    "efm_sage_quantize": (c_int32, [POINTER(AttentionCtx), c_void_p, c_void_p, c_uint32, c_uint32, c_void_p, c_void_p,
                                    c_void_p, c_void_p, c_void_p, c_void_p]),
    "efm_rope_llama_inplace": (c_int32, [c_void_p, c_void_p, c_int32, c_int32, c_int32, c_int32, c_int32, c_int32,
                                         c_int32, c_float, c_float, c_void_p]),
    "efm_mrope": (c_int32, [c_void_p, c_void_p, c_void_p, c_int32, c_int32, c_int32, c_int32, c_int32, c_int32,
                            c_int32, c_int32, c_int32, c_int32, c_float, c_float, c_void_p]),
    "efm_prefill_rope_write_kv": (c_int32, [c_void_p, c_int32, c_void_p, c_void_p, c_int32, c_int32, c_int32, c_int32,
                                            c_int32, c_void_p, c_int32, c_int32, c_int32, c_int32, c_int32, c_float,
                                            c_float, c_void_p]),
    "efm_decode_mrope_write_kv": (c_int32, [c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_int32,
                                            c_int32, c_int32, c_void_p, c_int32, c_int32, c_int32, c_float, c_float,
                                            c_void_p, c_void_p]),
    "efm_finalize_decode_token_indexed": (c_int32, [c_void_p, c_void_p, c_void_p, c_void_p, c_uint32, c_void_p]),
    "efm_rms_norm": (c_int32, [c_uint32, c_uint32, c_float, c_void_p, c_void_p, c_void_p, c_void_p]),
    "efm_fused_add_rms_norm": (c_int32, [c_uint32, c_uint32, c_float, c_void_p, c_void_p, c_void_p, c_void_p]),
    "efm_act_and_mul": (c_int32, [c_int64, c_int64, c_int32, c_void_p, c_void_p, c_void_p]),
    "efm_linear": (c_int32, [c_int64, c_int64, c_int64, c_void_p, c_void_p, c_void_p, c_void_p, c_int32, c_void_p]),
    "efm_linear_workspace_bytes": (c_size_t, [c_int64, c_int64, c_int64]),
    "efm_linear_ws": (c_int32, [c_int64, c_int64, c_int64, c_void_p, c_void_p, c_void_p, c_void_p, c_int32, c_void_p,
                                c_size_t, c_void_p]),
    "efm_fused_gate_up_swiglu": (c_int32, [c_int64, c_int64, c_int64, c_void_p, c_void_p, c_void_p, c_void_p]),
    "efm_fused_gate_up_swiglu_workspace_bytes": (c_size_t, [c_int64, c_int64, c_int64]),
    "efm_fused_gate_up_swiglu_ws": (c_int32, [c_int64, c_int64, c_int64, c_void_p, c_void_p, c_void_p, c_void_p,
                                              c_size_t, c_void_p]),
    "efm_testing_set_kernel_path": (c_int32, [c_int32, c_int32]),
    "efm_lm_head_top1_workspace_bytes": (c_size_t, [c_int64]),
    "efm_lm_head_top1": (c_int32, [c_int64, c_int64, c_void_p, c_void_p, c_void_p, c_void_p, c_size_t, c_void_p]),
    "efm_sampler_greedy_workspace_bytes": (c_size_t, [c_int64, c_int64]),
    "efm_sampler_greedy": (c_int32, [c_int64, c_int64, c_void_p, c_void_p, c_void_p, c_size_t, c_void_p]),
    "efm_sampler_top_p_workspace_bytes": (c_size_t, [c_int64]),
    "efm_sampler_top_p": (c_int32, [c_int64, c_void_p, c_float, c_float, c_uint64, c_uint64, c_void_p, c_void_p,
                                    c_void_p, c_size_t, c_void_p]),
    "efm_embedding_lookup": (c_int32, [c_int64, c_int64, c_int64, c_void_p, c_void_p, c_void_p, c_int64, c_int32,
                                       c_void_p, c_void_p]),
    "efm_copy_decode_kv_cache_slots": (c_int32, [c_void_p, c_void_p, c_void_p, c_void_p, c_int32, c_int32, c_void_p,
                                                 c_void_p]),
    "efm_finalize_decode_token": (c_int32, [c_void_p, c_void_p, c_void_p, c_void_p]),
    "efm_increment_int32_triplet": (c_int32, [c_void_p, c_void_p]),
    "efm_decode_norm_qkv": (c_int32, [c_int32, c_int32, c_int32, c_float, c_void_p, c_void_p, c_void_p, c_void_p,
                                      c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p]),
    "efm_store_row_indexed": (c_int32, [c_void_p, c_void_p, c_int64, c_void_p, c_uint32, c_void_p]),
    "efm_decode_norm_qkv_rope": (c_int32, [POINTER(AttentionCtx), c_int32, c_float, c_void_p, c_void_p, c_void_p,
                                           c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p,
                                           c_void_p]),
    "efm_decode_qkv_attention_sync_bytes": (c_size_t, [c_int32, c_int32]),
    "efm_decode_norm_qkv_attention_supported": (c_int32, [POINTER(AttentionCtx), c_int32, c_uint32]),
    "efm_decode_norm_qkv_attention": (c_int32, [POINTER(AttentionCtx), c_int32, c_float, c_void_p, c_void_p, c_void_p,
                                                c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_uint32,
                                                c_void_p, c_size_t, c_void_p, c_size_t, c_void_p]),
    "efm_decode_qkv_attention_status": (c_int32, [c_void_p, c_void_p]),
    "efm_decode_norm_gate_up_swiglu": (c_int32, [c_int32, c_int32, c_float, c_void_p, c_void_p, c_void_p, c_void_p,
                                                 c_void_p, c_void_p, c_void_p]),
    "efm_decode_norm_lm_head_top1": (c_int32, [c_int32, c_int64, c_float, c_void_p, c_void_p, c_void_p, c_void_p,
                                               c_void_p, c_void_p, c_size_t, c_void_p]),
}


class EfmError(RuntimeError):
    def __init__(self, code: int, message: str):
        super().__init__(f"edgefm_hip error {code}: {message}")
        self.code = code


_lib = None


def load(path: str = LIB_PATH) -> ctypes.CDLL:
    """Load the kernel library (once) and attach the prototypes."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(path):
        raise RuntimeError(f"edgefm_hip library not built: {path} is missing (run __graft_entry__.build())")
    # PyTorch-ROCm ships its own HIP runtime, loaded by file path: if this library were
    # loaded first it would bind /opt/rocm's copy and the process would hold two
    # runtimes whose device state does not mix. Loading torch first makes this library
    # resolve libamdhip64.so.7 to torch's already-loaded copy.
    try:
        import torch  # noqa: F401
    except ImportError:
        pass
    lib = ctypes.CDLL(path)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib


def call(name: str, *args) -> None:
    """Invoke an entry point returning a status code; raise EfmError on failure."""
    lib = load()
    rc = getattr(lib, name)(*args)
    if rc != EFM_OK:
        raise EfmError(rc, lib.efm_last_error().decode())
