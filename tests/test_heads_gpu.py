"""Head layouts other than the reference's 4 q/k heads and 8 v-heads, on the
GPU: decode (one token and several), and prefill through both paths (the
chunk-64 pipeline and the token-sequential kernel), against the oracle on the
same seeded inputs.

The reference fixes 4/8 heads in its definitions (gdn_decode_ref.py:32-34,
gdn_prefill_ref.py:31-33); the head count enters its algorithm only through
the GVA expansion (v-head h reads q/k head h // (HV / HQK),
gdn_decode_ref.py:57-58, gdn_prefill_ref.py:42-43).  The oracle's general-head
form is pinned on the CPU by tests/test_oracle.py (per-head problems and the
C vs numpy restatements).  Tolerance as everywhere (conftest.py): bf16 output
atol = rtol = 1e-2; f32 state atol = 1e-3 * max|state_ref|.
"""

import ctypes

import numpy as np
import pytest
import torch

from test_recurrent_gpu import _expected_multi_kind  # noqa: E402
from conftest import assert_output_close, assert_state_close
from oracle import gdn_oracle as O

pytestmark = pytest.mark.gpu

from gdn_amd import _lib, decode, prefill  # noqa: E402

# (q/k heads, v-heads): Qwen3-Next-like 16/32, GVA ratio 4, no GVA, one head.
HEADS = [(16, 32), (2, 8), (8, 8), (1, 1)]
ALL_SEQUENTIAL = 1 << 30


def _to_dev(inp, dev):
    bf = torch.bfloat16
    d = {n: torch.from_numpy(np.ascontiguousarray(inp[n])).to(dev).to(bf)
         for n in ("q", "k", "v", "a", "b")}
    for n in ("A_log", "dt_bias"):
        d[n] = torch.from_numpy(inp[n]).to(dev)
    d["state"] = None if inp["state"] is None else torch.from_numpy(inp["state"]).to(dev)
    if "cu_seqlens" in inp:
        d["cu_seqlens"] = torch.from_numpy(inp["cu_seqlens"]).to(dev)
    d["scale"] = inp["scale"]
    return d


def _decode(d, dev, variant=-1):
    B, T, hv = d["v"].shape[0], d["v"].shape[1], d["v"].shape[2]
    out = torch.empty((B, T, hv, 128), dtype=torch.bfloat16, device=dev)
    ns = torch.empty((B, hv, 128, 128), dtype=torch.float32, device=dev)
    decode.kernel(d["q"], d["k"], d["v"], d["state"], d["A_log"], d["a"], d["dt_bias"], d["b"],
                  d["scale"], out, ns, variant=variant)
    torch.cuda.synchronize()
    return out, ns


def _prefill(d, dev, rec_max):
    T, hv = d["v"].shape[0], d["v"].shape[1]
    N = d["cu_seqlens"].numel() - 1
    out = torch.empty((T, hv, 128), dtype=torch.bfloat16, device=dev)
    ns = torch.empty((N, hv, 128, 128), dtype=torch.float32, device=dev)
    prefill.kernel(d["q"], d["k"], d["v"], d["state"], d["A_log"], d["a"], d["dt_bias"], d["b"],
                   d["cu_seqlens"], d["scale"], out, ns, recurrent_max_len=rec_max)
    torch.cuda.synchronize()
    return out, ns


@pytest.mark.parametrize("heads", HEADS)
@pytest.mark.parametrize("B", [1, 33])
def test_decode_heads_matches_oracle(cuda_device, heads, B):
    print(f"decode heads={heads} B={B}", flush=True)
    inp = O.make_decode_inputs(B, seed=40 + B, heads=heads)
    out, ns = _decode(_to_dev(inp, cuda_device), cuda_device)
    o_ref, s_ref = O.decode(**inp)
    assert_output_close(out.float().cpu().numpy(), o_ref)
    assert_state_close(ns.cpu().numpy(), s_ref)


def _multi(heads, B, T, seed, with_state=True):
    inp = O.make_prefill_inputs([T] * B, seed=seed, heads=heads, with_state=with_state)
    hqk, hv = heads
    dec = dict(inp)
    for n, tail in (("q", (hqk, 128)), ("k", (hqk, 128)), ("v", (hv, 128)), ("a", (hv,)),
                    ("b", (hv,))):
        dec[n] = inp[n].reshape((B, T) + tail)
    del dec["cu_seqlens"]
    return inp, dec


@pytest.mark.parametrize("heads", HEADS)
def test_multi_token_decode_heads_matches_oracle(cuda_device, heads):
    B, T = 6, 5
    print(f"multi-token decode heads={heads} B={B} T={T}", flush=True)
    inp, dec = _multi(heads, B, T, seed=50)
    out, ns = _decode(_to_dev(dec, cuda_device), cuda_device)
    o_ref, s_ref = O.prefill_seq_c(**inp)
    assert_output_close(out.reshape(B * T, heads[1], 128).float().cpu().numpy(), o_ref)
    # token by token holds the f32 sequential bound; the block kernel (split
    # bf16 products) the parity tolerance
    token = _expected_multi_kind(B, T, hv=heads[1]) == "token"
    assert_state_close(ns.cpu().numpy(), s_ref, rel_atol=1e-5 if token else 1e-3)


@pytest.mark.parametrize("heads", HEADS)
def test_decode_heads_tilings_are_identical(cuda_device, heads):
    inp = O.make_decode_inputs(9, seed=41, heads=heads)
    d = _to_dev(inp, cuda_device)
    ref_o, ref_s = _decode(d, cuda_device, variant=0)
    for var in range(1, 10):
        o, s = _decode(d, cuda_device, variant=var)
        assert torch.equal(o, ref_o) and torch.equal(s, ref_s), f"tiling {var}"
    o_ref, s_ref = O.decode(**inp)
    assert_output_close(ref_o.float().cpu().numpy(), o_ref)
    assert_state_close(ref_s.cpu().numpy(), s_ref)


PREFILL_LENS = {
    "chunked": ([300, 64, 0, 129], -2),
    "sequential": ([6, 49, 0, 61], ALL_SEQUENTIAL),
    "auto": ([8, 700, 1, 40], -1),
}


@pytest.mark.parametrize("heads", HEADS)
@pytest.mark.parametrize("route", list(PREFILL_LENS))
def test_prefill_heads_matches_oracle(cuda_device, heads, route):
    lens, rec_max = PREFILL_LENS[route]
    print(f"prefill heads={heads} route={route} lens={lens}", flush=True)
    inp = O.make_prefill_inputs(lens, seed=60, heads=heads)
    out, ns = _prefill(_to_dev(inp, cuda_device), cuda_device, rec_max)
    o_ref, s_ref = O.prefill_seq_c(**inp)
    assert_output_close(out.float().cpu().numpy(), o_ref)
    assert_state_close(ns.cpu().numpy(), s_ref)
    assert not ns.cpu().numpy()[[i for i, n in enumerate(lens) if n == 0]].any()


def test_prefill_heads_single_long_sequence(cuda_device):
    heads = (16, 32)
    inp = O.make_prefill_inputs([1000], seed=61, heads=heads, with_state=False)
    out, ns = _prefill(_to_dev(inp, cuda_device), cuda_device, -1)
    o_ref, s_ref = O.prefill_seq_c(**inp)
    assert_output_close(out.float().cpu().numpy(), o_ref)
    assert_state_close(ns.cpu().numpy(), s_ref)


def test_prefill_heads_wy_product_form(cuda_device):
    # 1600 tokens at 32 v-heads: 25 chunks x 32 = 800 (chunk, v-head) units,
    # past the 768 from which the WY intra kernel forms w and u as T and two
    # products instead of two solves (one sequence: WY form, one chain)
    heads = (16, 32)
    inp = O.make_prefill_inputs([1600], seed=62, heads=heads, with_state=True)
    print(f"prefill heads={heads} lens=[1600] (product form)", flush=True)
    out, ns = _prefill(_to_dev(inp, cuda_device), cuda_device, -1)
    o_ref, s_ref = O.prefill_seq_c(**inp)
    assert_output_close(out.float().cpu().numpy(), o_ref)
    assert_state_close(ns.cpu().numpy(), s_ref)


def _ptr(t):
    return None if t is None else t.data_ptr()


def test_heads_entry_points_equal_fixed_ones_at_4_8(cuda_device):
    """gdn_decode_fwd_heads / gdn_prefill_fwd_heads called with 4 and 8 heads
    give bit-identical results to gdn_decode_fwd / gdn_prefill_fwd."""
    lib = _lib.load()
    stream = torch.cuda.current_stream(cuda_device).cuda_stream
    dev = cuda_device

    inp = O.make_decode_inputs(17, seed=42)
    d = _to_dev(inp, dev)
    o1, s1 = _decode(d, dev)
    o2, s2 = torch.empty_like(o1), torch.empty_like(s1)
    rc = lib.gdn_decode_fwd_heads(*(_ptr(d[n]) for n in ("q", "k", "v", "state", "A_log", "a",
                                                       "dt_bias", "b")),
                                  d["scale"], o2.data_ptr(), s2.data_ptr(), 17, 1, 4, 8, stream,
                                  -1)
    _lib.check(rc, "gdn_decode_fwd_heads")
    torch.cuda.synchronize()
    assert torch.equal(o1, o2) and torch.equal(s1, s2)

    for lens, rec_max in ((([300, 64, 0, 129]), -2), ([6, 49, 61], ALL_SEQUENTIAL)):
        inp = O.make_prefill_inputs(lens, seed=43)
        d = _to_dev(inp, dev)
        o1, s1 = _prefill(d, dev, rec_max)
        T, N = sum(lens), len(lens)
        nbytes = lib.gdn_prefill_workspace_bytes_heads(T, N, 4, 8)
        assert nbytes == lib.gdn_prefill_workspace_bytes(T, N)
        ws = torch.empty(max(nbytes, 256), dtype=torch.uint8, device=dev)
        o2, s2 = torch.empty_like(o1), torch.empty_like(s1)
        rc = lib.gdn_prefill_fwd_heads(
            *(_ptr(d[n]) for n in ("q", "k", "v", "state", "A_log", "a", "dt_bias", "b")),
            d["cu_seqlens"].data_ptr(), 1, N, T, 4, 8, d["scale"], o2.data_ptr(), s2.data_ptr(),
            ws.data_ptr(), ctypes.c_size_t(ws.numel()), stream, -1, rec_max, -1)
        _lib.check(rc, "gdn_prefill_fwd_heads")
        torch.cuda.synchronize()
        assert torch.equal(o1, o2) and torch.equal(s1, s2), f"lens={lens}"


def test_heads_rejects(cuda_device):
    """8 v-heads over 3 q/k heads is refused before any launch."""
    inp = O.make_decode_inputs(2, seed=44, heads=(3, 8))
    d = _to_dev(inp, cuda_device)
    with pytest.raises(ValueError, match="multiple"):
        _decode(d, cuda_device)
    inp = O.make_prefill_inputs([5, 7], seed=45, heads=(2, 8))
    d = _to_dev(inp, cuda_device)
    d["q"] = torch.cat([d["q"], d["q"][:, :1]], dim=1)  # 3 q/k heads
    d["k"] = torch.cat([d["k"], d["k"][:, :1]], dim=1)
    with pytest.raises(ValueError, match="multiple"):
        _prefill(d, cuda_device, -1)
