"""The cu_seqlens status words every prefill call leaves in its workspace.

Contract (include/gdn_amd.h, gdn_prefill_status_offset): the offsets are
non-decreasing and within [0, T].  A call with N >= 1 writes, on the device,
one word per sequence -- bit 0 if cu[s+1] < cu[s], bit 1 if cu[s] or cu[s+1]
is outside [0, T] -- in the first kernel that reads the bounds: the index
kernel, the intra kernel's own scan, the single sequence's intra kernel, or a
sequential kernel the host routed the batch to.  The reference has no such
check: it reads the bounds on the host and skips a sequence whose length is
not positive (reference/gdn_prefill_ref.py:55-61).

Well-formed batches must read 0 on every path; malformed ones the bits they
break.  Their outputs are unspecified by the contract, but every kernel
clamps the bounds it reads into [0, T] (load_cu, the chunk table's clamps to
the chunk slots), so a malformed batch computes over in-range tokens only --
these calls check that the call completes and the status, not the outputs.
Well-formed cases also match the oracle, as in every parity test
(conftest.py tolerances).
"""

import ctypes

import numpy as np
import pytest
import torch

from conftest import assert_output_close, assert_state_close
from oracle import gdn_oracle as O

pytestmark = pytest.mark.gpu

from gdn_amd import _lib, prefill  # noqa: E402


def _even(T, N):
    return [round(T * i / N) for i in range(N + 1)]


def _swap(cu, i):
    cu = list(cu)
    cu[i], cu[i + 1] = cu[i + 1], cu[i]
    return cu


def _set(cu, i, x):
    cu = list(cu)
    cu[i] = x
    return cu


# name -> (T, cu_seqlens, expected bits).  The paths: one sequence through the
# chunks (its intra kernel writes the word) or sequentially (T <= 96); a few
# short sequences routed sequentially on the host; a few sequences through
# the chunks with the intra kernel's own scan; 64 x 16 tokens (the device
# picks the path, the intra kernel's scan); 300 sequences (the index kernel);
# 6 x 4096 tokens (more intra workgroups than the intra scan takes: the index
# kernel).
CASES = {
    "one_chunks": (1000, [0, 1000], 0),
    "one_chunks_decreasing": (1000, [300, 200], 1),
    "one_chunks_negative": (1000, [-4, 900], 2),
    "one_chunks_past_T": (1000, [0, 1100], 2),
    "one_short": (60, [0, 60], 0),
    "one_short_past_T": (60, [0, 70], 2),
    "one_short_decreasing": (60, [50, 10], 1),
    "host_seq": (90, [0, 30, 60, 90], 0),
    "host_seq_decreasing": (90, [0, 50, 40, 90], 1),
    "host_seq_both": (90, [0, 50, 40, 95], 3),
    "self_index": (1200, [0, 300, 800, 1200], 0),
    "self_index_decreasing": (1200, [0, 800, 300, 1200], 1),
    "self_index_past_T": (1200, [0, 300, 800, 1300], 2),
    "device_choice": (1024, _even(1024, 64), 0),
    "device_choice_decreasing": (1024, _swap(_even(1024, 64), 10), 1),
    "device_choice_negative": (1024, _set(_even(1024, 64), 0, -16), 2),
    "index_kernel": (3000, _even(3000, 300), 0),
    "index_kernel_decreasing": (3000, _swap(_even(3000, 300), 150), 1),
    "index_kernel_past_T": (3000, _set(_even(3000, 300), 300, 3001), 2),
    "index_kernel_large": (24576, _even(24576, 6), 0),
    "index_kernel_large_decreasing": (24576, _swap(_even(24576, 6), 3), 1),
}


def _inputs(T, cu, seed, int64):
    inp = O.make_prefill_inputs([T], seed=seed, with_state=False)
    N = len(cu) - 1
    rng = np.random.default_rng(seed + 1)
    inp["state"] = (0.05 * rng.standard_normal((N, 8, 128, 128))).astype(np.float32)
    inp["cu_seqlens"] = np.asarray(cu, dtype=np.int64 if int64 else np.int32)
    return inp


def _to_dev(inp, dev):
    bf = torch.bfloat16
    d = {n: torch.from_numpy(np.ascontiguousarray(inp[n])).to(dev).to(bf)
         for n in ("q", "k", "v", "a", "b")}
    for n in ("A_log", "dt_bias", "state", "cu_seqlens"):
        d[n] = torch.from_numpy(inp[n]).to(dev)
    return d


@pytest.mark.parametrize("name", list(CASES))
def test_status_words(cuda_device, name):
    dev = cuda_device
    T, cu, want = CASES[name]
    N = len(cu) - 1
    int64 = len(name) % 2 == 0  # both index widths across the cases
    print(f"status {name}: T={T} N={N} int64={int64} expect {want}", flush=True)
    inp = _inputs(T, cu, seed=len(name), int64=int64)
    d = _to_dev(inp, dev)
    out = torch.empty((T, 8, 128), dtype=torch.bfloat16, device=dev)
    ns = torch.empty((N, 8, 128, 128), dtype=torch.float32, device=dev)
    prefill.kernel(d["q"], d["k"], d["v"], d["state"], d["A_log"], d["a"], d["dt_bias"], d["b"],
                   d["cu_seqlens"], inp["scale"], out, ns)
    assert prefill.batch_status(T, N) == want
    if want == 0:
        o_ref, s_ref = O.prefill_seq_c(**inp)
        assert_output_close(out.float().cpu().numpy(), o_ref)
        assert_state_close(ns.cpu().numpy(), s_ref)


def test_status_is_rewritten_by_every_call(cuda_device):
    # a malformed call, then a well-formed one of the same (T, N): the second
    # leaves 0 (each call writes every word), and back
    dev = cuda_device
    T = 1200
    for cu, want in (([0, 800, 300, 1200], 1), ([0, 300, 800, 1200], 0), ([0, 300, 800, 1300], 2)):
        inp = _inputs(T, cu, seed=5, int64=False)
        d = _to_dev(inp, dev)
        out = torch.empty((T, 8, 128), dtype=torch.bfloat16, device=dev)
        ns = torch.empty((3, 8, 128, 128), dtype=torch.float32, device=dev)
        prefill.kernel(d["q"], d["k"], d["v"], d["state"], d["A_log"], d["a"], d["dt_bias"],
                       d["b"], d["cu_seqlens"], inp["scale"], out, ns)
        assert prefill.batch_status(T, 3) == want, cu


def test_status_of_the_allocation_free_entry_point(cuda_device):
    # gdn_prefill_status with workspace NULL reads the static scratch
    dev = cuda_device
    lib = _lib.load()
    stream = torch.cuda.current_stream(dev).cuda_stream
    T = 1200
    for cu, want in (([0, 800, 300, 1200], 1), ([0, 300, 800, 1200], 0)):
        inp = _inputs(T, cu, seed=9, int64=True)
        d = _to_dev(inp, dev)
        out = torch.empty((T, 8, 128), dtype=torch.bfloat16, device=dev)
        ns = torch.empty((3, 8, 128, 128), dtype=torch.float32, device=dev)
        rc = lib.gdn_prefill_fwd_noalloc(
            d["q"].data_ptr(), d["k"].data_ptr(), d["v"].data_ptr(), d["state"].data_ptr(),
            d["A_log"].data_ptr(), d["a"].data_ptr(), d["dt_bias"].data_ptr(), d["b"].data_ptr(),
            d["cu_seqlens"].data_ptr(), 1, 3, T, float(inp["scale"]), out.data_ptr(),
            ns.data_ptr(), stream)
        _lib.check(rc, "gdn_prefill_fwd_noalloc")
        got = ctypes.c_int(-1)
        rc = lib.gdn_prefill_status(None, T, 3, 4, 8, stream, ctypes.byref(got))
        _lib.check(rc, "gdn_prefill_status")
        assert got.value == want, cu


@pytest.mark.parametrize("rec_max", [-2, -1])
def test_status_of_a_call_without_tokens(cuda_device, rec_max):
    # T = 0 and one sequence: through the chunks (-2) no intra kernel runs, so
    # the status word has a launch of its own; a stale word from the previous
    # call of the same (T, N) must not survive.
    dev = cuda_device
    print(f"status T=0 N=1 rec_max={rec_max}", flush=True)
    for cu, want in (([0, 5], 2), ([0, 0], 0), ([3, 1], 3), ([0, 0], 0)):
        inp = _inputs(0, cu, seed=11, int64=True)
        d = _to_dev(inp, dev)
        out = torch.empty((0, 8, 128), dtype=torch.bfloat16, device=dev)
        ns = torch.full((1, 8, 128, 128), 7.0, dtype=torch.float32, device=dev)
        prefill.kernel(d["q"], d["k"], d["v"], d["state"], d["A_log"], d["a"], d["dt_bias"],
                       d["b"], d["cu_seqlens"], inp["scale"], out, ns, recurrent_max_len=rec_max)
        assert prefill.batch_status(0, 1) == want, cu
        if want == 0:  # a zero-length sequence: zero state (gdn_prefill_ref.py:61-62)
            assert not ns.cpu().numpy().any()
