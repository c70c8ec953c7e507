"""Helpers shared by the GPU parity tests: raw pointers and the current HIP stream."""
import torch


def ptr(t):
    return None if t is None else t.data_ptr()


def stream():
    return torch.cuda.current_stream().cuda_stream


def bf16_tol():
    # tests/operators/_test_utils.py:171-176 (bf16 rtol/atol 1e-2)
    return dict(rtol=1e-2, atol=1e-2)


def assert_close_bf16(out, ref, rtol=1e-2, atol=1e-2, what=""):
    o = out.detach().float().cpu()
    r = ref.detach().float().cpu()
    torch.testing.assert_close(o, r, rtol=rtol, atol=atol, msg=lambda m: f"{what}: {m}")
