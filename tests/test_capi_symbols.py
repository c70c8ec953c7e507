"""CPU test: the C-ABI library loads and exports every entry point include/*.h
declares, and the ctypes binding declares exactly the same set (no compute calls)."""
import ctypes
import glob
import os
import re

import efm_capi as C

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _declared():
    names = set()
    for h in glob.glob(os.path.join(ROOT, "include", "*.h")):
        text = open(h).read()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        names |= set(re.findall(r"\b(efm_[a-z0-9_]+)\s*\(", text))
    return names


def test_library_exports_every_declared_symbol():
    lib = ctypes.CDLL(C.LIB_PATH)
    declared = _declared()
    assert len(declared) >= 20
    missing = [n for n in sorted(declared) if not hasattr(lib, n)]
    assert not missing, f"declared but not exported: {missing}"


def test_ctypes_binding_covers_header():
    assert set(C.SIGNATURES) == _declared()


def test_version_and_error_strings():
    lib = C.load()
    assert lib.efm_version().decode().startswith("edgefm-hip")
    assert isinstance(lib.efm_last_error(), bytes)


def test_host_side_validation_without_gpu():
    """Argument checks run on the host before any launch, so they work without a GPU."""
    lib = C.load()
    ctx = C.make_attention_ctx(10, 2, 128)  # GQA group 5: unsupported (attention_op.cu:41)
    rc = lib.efm_attention_decode(ctx, 1, 1, 1, 1, 1, None, 0, 1, 1 << 20, None)
    assert rc == C.EFM_ERR_UNSUPPORTED and b"group size" in lib.efm_last_error()
    rc = lib.efm_linear(1, 1530, 8, 16, 16, None, 16, C.EFM_DTYPE_BF16, None)
    assert rc == C.EFM_ERR_UNSUPPORTED
    assert lib.efm_attention_decode_workspace_bytes(C.make_attention_ctx(12, 2, 128), 4096) > 0


def test_gemm_workspace_queries_without_gpu():
    """The split-K plan, and so the workspace query, depends on the shape alone: long-K
    shapes with few output tiles use a workspace; shapes that fill the chip, and the
    SwiGLU GEMM (its activation is the MFMA epilogue), use none. The library links no
    vendor GEMM library."""
    lib = C.load()
    assert lib.efm_linear_workspace_bytes(1344, 11008, 2048) == 0
    assert lib.efm_linear_workspace_bytes(512, 8960, 1536) > 0
    assert lib.efm_linear_workspace_bytes(1, 8960, 1536) == 0
    assert lib.efm_fused_gate_up_swiglu_workspace_bytes(512, 1536, 8960) == 0
    assert not hasattr(lib, "efm_set_gemm_backend")
    with open(C.LIB_PATH, "rb") as f:
        assert b"libhipblaslt" not in f.read()


def test_testing_kernel_path_setter_validates():
    """The test-only kernel-path knobs accept their documented values, reject others, and
    reset to the library's own choice (0)."""
    lib = C.load()
    assert lib.efm_testing_set_kernel_path(C.EFM_KNOB_DECODE_REGISTER, 1) == C.EFM_OK
    assert lib.efm_testing_set_kernel_path(C.EFM_KNOB_DECODE_REGISTER, 0) == C.EFM_OK
    assert lib.efm_testing_set_kernel_path(C.EFM_KNOB_PREFILL_SHAPE, 8) == C.EFM_OK
    assert lib.efm_testing_set_kernel_path(C.EFM_KNOB_PREFILL_SHAPE, 2) == C.EFM_OK
    assert lib.efm_testing_set_kernel_path(C.EFM_KNOB_PREFILL_SHAPE, 0) == C.EFM_OK
    assert lib.efm_testing_set_kernel_path(C.EFM_KNOB_PREFILL_SHAPE, 5) == C.EFM_ERR_INVALID_ARGUMENT
    assert lib.efm_testing_set_kernel_path(C.EFM_KNOB_PREFILL_REGISTER, 2) == C.EFM_ERR_INVALID_ARGUMENT
    assert lib.efm_testing_set_kernel_path(C.EFM_KNOB_GEMM_TILE, 2) == C.EFM_OK
    assert lib.efm_testing_set_kernel_path(C.EFM_KNOB_GEMM_TILE, 0) == C.EFM_OK
    assert lib.efm_testing_set_kernel_path(C.EFM_KNOB_GEMM_TILE, 3) == C.EFM_OK
    assert lib.efm_testing_set_kernel_path(C.EFM_KNOB_GEMM_TILE, 0) == C.EFM_OK
    assert lib.efm_testing_set_kernel_path(C.EFM_KNOB_GEMM_TILE, 4) == C.EFM_ERR_INVALID_ARGUMENT
    assert lib.efm_testing_set_kernel_path(C.EFM_KNOB_FRONT_WAIT_TIMEOUT, 1) == C.EFM_OK
    assert lib.efm_testing_set_kernel_path(C.EFM_KNOB_FRONT_WAIT_TIMEOUT, 0) == C.EFM_OK
    assert lib.efm_testing_set_kernel_path(C.EFM_KNOB_FRONT_WAIT_TIMEOUT, 2) == C.EFM_ERR_INVALID_ARGUMENT
    assert lib.efm_testing_set_kernel_path(C.EFM_KNOB_DECODE_TILE, 1) == C.EFM_OK
    assert lib.efm_testing_set_kernel_path(C.EFM_KNOB_DECODE_TILE, 0) == C.EFM_OK
    assert lib.efm_testing_set_kernel_path(C.EFM_KNOB_DECODE_TILE, 2) == C.EFM_ERR_INVALID_ARGUMENT
    assert lib.efm_testing_set_kernel_path(6, 0) == C.EFM_ERR_INVALID_ARGUMENT
    assert lib.efm_testing_set_kernel_path(99, 0) == C.EFM_ERR_INVALID_ARGUMENT


def test_merge_o_proj_plan_query_without_gpu():
    """The partials plan that efm_decode_attention_merge_o_proj reads back: query widths up
    to 1024 merge up to 24 splits, widths up to 2048 up to 12 (splits of 32 / 64 keys from
    the one-wave kernel where they fit, else of 128 keys)."""
    lib = C.load()
    sup = lib.efm_decode_attention_merge_o_proj_supported
    assert sup(C.make_attention_ctx(14, 2, 64), 1025) == C.EFM_OK          # 17 splits of 64 keys
    assert sup(C.make_attention_ctx(16, 2, 64), 1536) == C.EFM_OK          # 24 splits of 64 keys
    assert sup(C.make_attention_ctx(14, 2, 64), 3072) == C.EFM_OK          # 24 splits of 128 keys
    assert sup(C.make_attention_ctx(14, 2, 64), 3073) == C.EFM_ERR_UNSUPPORTED
    assert sup(C.make_attention_ctx(32, 8, 64), 1536) == C.EFM_OK          # width 2048: 12 of 128
    assert sup(C.make_attention_ctx(32, 8, 64), 1537) == C.EFM_ERR_UNSUPPORTED
    assert sup(C.make_attention_ctx(12, 2, 128), 768) == C.EFM_OK          # 12 splits of 64 keys
    assert sup(C.make_attention_ctx(12, 2, 128), 1536) == C.EFM_OK
    assert sup(C.make_attention_ctx(12, 2, 128), 1537) == C.EFM_ERR_UNSUPPORTED
    assert sup(C.make_attention_ctx(28, 4, 128), 64) == C.EFM_ERR_UNSUPPORTED   # width 3584
    assert sup(C.make_attention_ctx(14, 2, 64), 0) == C.EFM_ERR_INVALID_ARGUMENT
    # the one-wave plan's splits fit the workspace the size query reports
    ctx = C.make_attention_ctx(14, 2, 64)
    assert lib.efm_attention_decode_workspace_bytes(ctx, 1536) >= 2 * 24 * 7 * 64 * 4 + 2 * 24 * 7 * 2 * 4
    ctx = C.make_attention_ctx(12, 2, 128)
    assert lib.efm_attention_decode_workspace_bytes(ctx, 768) >= 2 * 12 * 6 * 128 * 4 + 2 * 12 * 6 * 2 * 4
