"""Host-side logic of the Python entry points (no GPU needed): argument
resolution and validation happen before anything reaches the C ABI."""

import math

import pytest
import torch

from gdn_amd import _common, decode, prefill


def test_resolve_scale_follows_reference():
    assert _common.resolve_scale(None) == 1 / math.sqrt(128)
    assert _common.resolve_scale(0.0) == 1 / math.sqrt(128)
    assert _common.resolve_scale(torch.tensor(0.5)) == 0.5
    assert _common.resolve_scale(2) == 2.0
    for bad in (-1.0, float("inf"), float("nan")):
        with pytest.raises(ValueError):
            _common.resolve_scale(bad)


def _decode_cpu_args(B=2):
    bf, f = torch.bfloat16, torch.float32
    return [torch.zeros(B, 1, 4, 128, dtype=bf), torch.zeros(B, 1, 4, 128, dtype=bf),
            torch.zeros(B, 1, 8, 128, dtype=bf), torch.zeros(B, 8, 128, 128, dtype=f),
            torch.zeros(8, dtype=f), torch.zeros(B, 1, 8, dtype=bf), torch.zeros(8, dtype=f),
            torch.zeros(B, 1, 8, dtype=bf), 1.0, torch.zeros(B, 1, 8, 128, dtype=bf),
            torch.zeros(B, 8, 128, 128, dtype=f)]


def test_decode_rejects_host_tensors():
    with pytest.raises(ValueError, match="device"):
        decode.kernel(*_decode_cpu_args())


def test_decode_rejects_bad_shapes_before_device_check():
    args = _decode_cpu_args()
    args[0] = torch.zeros(2, 4, 128, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="q must be"):
        decode.kernel(*args)


def test_prefill_rejects_host_tensors_and_bad_cu():
    bf, f = torch.bfloat16, torch.float32
    T = 10
    args = [torch.zeros(T, 4, 128, dtype=bf), torch.zeros(T, 4, 128, dtype=bf),
            torch.zeros(T, 8, 128, dtype=bf), None, torch.zeros(8, dtype=f),
            torch.zeros(T, 8, dtype=bf), torch.zeros(8, dtype=f), torch.zeros(T, 8, dtype=bf),
            torch.tensor([0, T]), 1.0, torch.zeros(T, 8, 128, dtype=bf),
            torch.zeros(1, 8, 128, 128, dtype=f)]
    with pytest.raises(ValueError, match="device"):
        prefill.kernel(*args)


def test_fast_ok_rejects_non_tensors_and_mismatches():
    t = torch.zeros(2, 3)
    assert not _common.fast_ok((t,), (torch.float32,), ((2, 3),))  # host tensor
    assert not _common.fast_ok((None,), (torch.float32,), ((2, 3),))
