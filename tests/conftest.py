"""Shared pytest set-up: import paths, the ``gpu`` marker and tolerances."""

import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "gated-delta-network_amd")
for p in (ROOT, PKG):
    if p not in sys.path:
        sys.path.insert(0, p)

# Parity bar of the operators (stated once, used by every parity test):
#   bf16 output: atol = rtol = 1e-2;  f32 state: atol = 1e-3 * max|state_ref|.
O_ATOL = 1e-2
O_RTOL = 1e-2
STATE_REL_ATOL = 1e-3


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (HIP device) and the built library")


def assert_output_close(got, ref, atol=O_ATOL, rtol=O_RTOL, what="output"):
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    assert got.shape == ref.shape, (got.shape, ref.shape)
    assert np.isfinite(got).all(), f"{what}: non-finite values"
    err = np.abs(got - ref)
    bad = err > atol + rtol * np.abs(ref)
    assert not bad.any(), (f"{what}: {int(bad.sum())} of {bad.size} elements out of tolerance; "
                           f"max abs err {err.max():.3e}")


def assert_state_close(got, ref, rel_atol=STATE_REL_ATOL, what="state"):
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    assert got.shape == ref.shape, (got.shape, ref.shape)
    assert np.isfinite(got).all(), f"{what}: non-finite values"
    scale = max(np.abs(ref).max(), 1e-30)
    err = np.abs(got - ref).max()
    assert err <= rel_atol * scale, f"{what}: max abs err {err:.3e} > {rel_atol:g} * {scale:.3e}"


@pytest.fixture(scope="session")
def cuda_device():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no HIP device visible")
    return torch.device("cuda", 0)
