"""Golden fixtures (tests/golden/, written by tests/golden/make_golden.py).

CPU: the seeded inputs still hash to the recorded SHA-256 and the oracle still
reproduces the stored outputs.  GPU: the HIP path matches the stored outputs
to the parity tolerance of conftest.py.
"""

import os

import numpy as np
import pytest

from conftest import assert_output_close, assert_state_close
from oracle import gdn_oracle as O

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def _load(name):
    import importlib.util
    spec = importlib.util.spec_from_file_location("make_golden", os.path.join(HERE, "make_golden.py"))
    mg = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mg)
    return mg, dict(np.load(os.path.join(HERE, name), allow_pickle=False))


def _decode_case():
    mg, fx = _load("decode_b1_seed0.npz")
    inp = O.make_decode_inputs(int(fx["B"]), seed=int(fx["seed"]))
    assert mg.input_digest(inp) == str(fx["sha256"]), "input generator changed"
    return inp, fx


def _prefill_case():
    mg, fx = _load("prefill_5_0_70_seed0.npz")
    inp = O.make_prefill_inputs(fx["lens"].tolist(), seed=int(fx["seed"]), with_state=False)
    assert mg.input_digest(inp) == str(fx["sha256"]), "input generator changed"
    return inp, fx


def _check_state(s_full, fx, seq=0):
    heads = fx["state_heads"]
    assert_state_close(s_full[seq, heads], fx["state_sel"])
    rs = s_full.astype(np.float64).sum(-1)
    # a row sum adds 128 entries: allow 128x the per-element bound
    lim = 128 * 1e-3 * np.abs(fx["state_sel"]).max()
    assert np.abs(rs - fx["state_rowsum"]).max() <= lim


def test_golden_decode_oracle():
    inp, fx = _decode_case()
    o, s = O.decode(**inp)
    assert np.array_equal(o, fx["o"])
    assert np.abs(s[0, fx["state_heads"]] - fx["state_sel"]).max() < 1e-6
    assert np.abs(s.astype(np.float64).sum(-1) - fx["state_rowsum"]).max() < 1e-4


def test_golden_prefill_oracle():
    inp, fx = _prefill_case()
    o, s = O.prefill_seq(**inp)
    assert np.array_equal(O.bf16_bits(o), fx["o_bits"])
    assert np.array_equal(s[int(fx["state_seq"]), fx["state_heads"]], fx["state_sel"])
    o2, s2 = O.prefill_seq_c(**inp)
    assert_output_close(o2, O.bf16_from_bits(fx["o_bits"]))
    _check_state(s2, fx, seq=int(fx["state_seq"]))


@pytest.mark.gpu
def test_golden_decode_gpu(cuda_device):
    import torch
    from gdn_amd import decode
    from test_decode_gpu import to_dev
    inp, fx = _decode_case()
    d = to_dev(inp, cuda_device)
    out = torch.empty((1, 1, 8, 128), dtype=torch.bfloat16, device=cuda_device)
    ns = torch.empty((1, 8, 128, 128), dtype=torch.float32, device=cuda_device)
    decode.kernel(d["q"], d["k"], d["v"], d["state"], d["A_log"], d["a"], d["dt_bias"], d["b"],
                  d["scale"], out, ns)
    torch.cuda.synchronize()
    assert_output_close(out.float().cpu().numpy(), fx["o"])
    _check_state(ns.cpu().numpy(), fx)


@pytest.mark.gpu
def test_golden_prefill_gpu(cuda_device):
    from test_prefill_gpu import run_gpu, to_dev
    inp, fx = _prefill_case()
    o, s = run_gpu(to_dev(inp, cuda_device), cuda_device)
    assert_output_close(o, O.bf16_from_bits(fx["o_bits"]))
    _check_state(s, fx, seq=int(fx["state_seq"]))
    assert np.all(s[1] == 0.0)
