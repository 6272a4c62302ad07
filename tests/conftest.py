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


# Output bound at large magnitudes for paths whose output products take
# single bf16 operands (the chunk pipeline's h and v_new, as in the
# reference's own chunk kernels, and the block kernel's P v_new).  Where atol
# no longer covers, the elementwise 1e-2 is about one bf16 ulp of the output
# (up to 2^-7 relative) plus 0.2 %, while two bf16-rounded operands add up to
# 2 * 2^-9: ~1.18e-2 of |o| in the worst case (1.15e-2 measured).  Those
# paths are held to |o - o_ref| <= 1.5e-2 * max|o_ref| per (token, head)
# row instead, on inputs whose state grows past ~1e20 (the reference's
# adversarial family) only.
ROW_REL = 1.5e-2


def assert_output_close_to_row_max(got, ref, rel=ROW_REL, what="output"):
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    assert got.shape == ref.shape, (got.shape, ref.shape)
    assert np.isfinite(got).all(), f"{what}: non-finite values"
    row_max = np.maximum(np.abs(ref).max(axis=-1, keepdims=True), 1e-30)
    worst = float((np.abs(got - ref) / row_max).max())
    assert worst <= rel, f"{what}: error {worst:.3e} of its row's max |o| > {rel:g}"


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
