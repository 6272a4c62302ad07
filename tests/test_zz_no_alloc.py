"""The allocation-free prefill entry point (gdn_prefill_fwd_noalloc) against
gdn_prefill_fwd with a caller-owned workspace, both through the C ABI.

Both run the same kernels on the same inputs, so their results must be equal
bit for bit; each is also checked against the CPU oracle at the parity
tolerance (bf16 output atol = rtol = 1e-2, f32 state 1e-3 * max|state_ref|).
The calls come in a row on one GPU -- a large batch, then a smaller one (the
static scratch keeps the first call's contents), then another large one -- so
leftovers of an earlier call must not leak into a later one.  Sizes beyond
the static maximum are refused before any device work.
"""

import ctypes

import numpy as np
import pytest
import torch

from conftest import assert_output_close, assert_state_close
from oracle import gdn_oracle as O

pytestmark = pytest.mark.gpu

from gdn_amd import _lib  # noqa: E402

# (lengths, seed): one sequence long enough for the two-segment scan, then a
# smaller packed batch (device-built chunk index), then a large one again.
CALLS = [
    ([3000], 90),
    ([6, 49, 294, 61, 100], 91),
    ([900, 1200, 1000], 92),
]


def _dev_inputs(inp, dev):
    bf = torch.bfloat16
    d = {n: torch.from_numpy(np.ascontiguousarray(inp[n])).to(dev).to(bf)
         for n in ("q", "k", "v", "a", "b")}
    for n in ("A_log", "dt_bias", "state", "cu_seqlens"):
        d[n] = torch.from_numpy(inp[n]).to(dev)
    return d


def _ptrs(d, out, ns):
    return (d["q"].data_ptr(), d["k"].data_ptr(), d["v"].data_ptr(), d["state"].data_ptr(),
            d["A_log"].data_ptr(), d["a"].data_ptr(), d["dt_bias"].data_ptr(), d["b"].data_ptr(),
            d["cu_seqlens"].data_ptr(), 1)


def test_noalloc_matches_workspace_entry_point(cuda_device):
    dev = cuda_device
    lib = _lib.load()
    stream = torch.cuda.current_stream(dev).cuda_stream
    for lens, seed in CALLS:
        T, N = sum(lens), len(lens)
        print(f"noalloc lens={lens} T={T} N={N}", flush=True)
        assert lib.gdn_prefill_workspace_bytes(T, N) <= _lib.PREFILL_SCRATCH_BYTES
        inp = O.make_prefill_inputs(lens, seed=seed)
        d = _dev_inputs(inp, dev)
        scale = float(inp["scale"])
        out_a = torch.full((T, 8, 128), 3.0, dtype=torch.bfloat16, device=dev)
        ns_a = torch.full((N, 8, 128, 128), 5.0, dtype=torch.float32, device=dev)
        rc = lib.gdn_prefill_fwd_noalloc(*_ptrs(d, out_a, ns_a), N, T, scale, out_a.data_ptr(),
                                         ns_a.data_ptr(), stream)
        _lib.check(rc, "gdn_prefill_fwd_noalloc")
        ws = torch.empty(lib.gdn_prefill_workspace_bytes(T, N), dtype=torch.uint8, device=dev)
        out_b = torch.empty_like(out_a)
        ns_b = torch.empty_like(ns_a)
        rc = lib.gdn_prefill_fwd(*_ptrs(d, out_b, ns_b), N, T, scale, out_b.data_ptr(),
                                 ns_b.data_ptr(), ws.data_ptr(), ws.numel(), stream)
        _lib.check(rc, "gdn_prefill_fwd")
        torch.cuda.synchronize()
        assert torch.equal(out_a, out_b), "output differs from gdn_prefill_fwd's"
        assert torch.equal(ns_a, ns_b), "new_state differs from gdn_prefill_fwd's"
        o_ref, s_ref = O.prefill_seq_c(**inp)
        assert_output_close(out_a.float().cpu().numpy(), o_ref)
        assert_state_close(ns_a.cpu().numpy(), s_ref)


def test_noalloc_refuses_batches_beyond_the_scratch(cuda_device):
    lib = _lib.load()
    T, N = 8192, 1
    assert lib.gdn_prefill_workspace_bytes(T, N) > _lib.PREFILL_SCRATCH_BYTES
    p = ctypes.c_void_p(1 << 20)
    rc = lib.gdn_prefill_fwd_noalloc(p, p, p, None, p, p, p, p, p, 1, N, T, 0.1, p, p, None)
    assert rc == _lib.GDN_ERR_WORKSPACE
    assert "static scratch" in _lib.last_error()
