"""Test configuration: registers the `gpu` marker and puts the repo root (oracle/),
the package directory (efm_capi, edge_fm) on sys.path."""
import os
import sys

import pytest
# before any test module imports edge_fm / loads libedgefm_hip.so: one HIP runtime per
# process (torch's), see efm_capi.load
import torch  # noqa: F401

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "edge-fm-x_amd")
for p in (ROOT, PKG):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built HIP library")


@pytest.fixture(scope="session")
def gpu():
    import torch

    if not torch.cuda.is_available():
        pytest.fail("GPU test selected but no GPU is visible")
    torch.cuda.set_device(0)
    return torch.device("cuda:0")


@pytest.fixture
def knob():
    """Setter for the library's test-only kernel-path knobs (efm_testing_set_kernel_path);
    every knob returns to the library's own choice (0) after the test."""
    import efm_capi as C

    def set_knob(which, value):
        C.call("efm_testing_set_kernel_path", which, int(value))

    yield set_knob
    for k in (C.EFM_KNOB_DECODE_REGISTER, C.EFM_KNOB_PREFILL_REGISTER, C.EFM_KNOB_PREFILL_SHAPE, C.EFM_KNOB_GEMM_TILE,
              C.EFM_KNOB_FRONT_WAIT_TIMEOUT, C.EFM_KNOB_DECODE_TILE):
        C.call("efm_testing_set_kernel_path", k, 0)
