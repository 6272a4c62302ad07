"""Prefill of packed buffers whose cu_seqlens do not span [0, T).

The reference zero-fills its output, runs sequence s over exactly the tokens
[cu[s], cu[s+1]) and leaves every other row at zero
(reference/gdn_prefill_ref.py:49-62); its FLA kernels honour cu_seqlens for a
single sequence too (solutions/gdn_prefill_qk4_v8_d128_k_last/solution/triton/
fla_kernels.py:959-972).  So a padded buffer (T = 128 holding one sequence
of 100 tokens, or one starting at token 20) must give the state after the
sequence's own tokens and zero rows elsewhere, on every path: the chunk
pipeline (one chain, the two-segment scan, both operand forms), the
token-by-token kernel and the 16-token block kernel, and under HIP-graph
replay with new cu_seqlens contents.

The output buffer is filled with a non-zero pattern before each call, so a
row the kernels leave unwritten fails the test.  Tolerances as every parity
test (conftest.py): bf16 output atol = rtol = 1e-2, f32 state atol =
1e-3 * max|state_ref|; uncovered rows must be exactly zero.
"""

import numpy as np
import pytest
import torch

from conftest import assert_output_close, assert_state_close
from oracle import gdn_oracle as O

pytestmark = pytest.mark.gpu

from gdn_amd import prefill  # noqa: E402

# (T, cu_seqlens): padded tails, a leading gap, both, gaps around an empty
# sequence, and single sequences in buffers long enough for the two-segment
# scan (whose split point comes from the chunk slots of T, so the sequence
# may end before or at the second segment).
CASES = [
    (128, [0, 100]),
    (256, [0, 100, 200]),
    (128, [20, 90]),
    (300, [7, 7, 150, 290]),
    (200, [64, 64]),
    (2500, [0, 2100]),
    (2500, [130, 2480]),
    (8192, [100, 5100]),
    (1000, [0, 100]),     # 16 chunk slots: the two-segment scan, its second segment empty
    (1000, [900, 1000]),
    (1000, [40, 640]),    # the sequence ends exactly at the second segment's first chunk
]

# name -> keyword arguments of prefill.kernel
ROUTES = {
    "auto": {},
    "chunks": dict(recurrent_max_len=-2),
    "chunks_one_chain": dict(recurrent_max_len=-2, variant=2),
    "chunks_two_segments": dict(recurrent_max_len=-2, variant=3),
    # the early output of the first segment cut short: the output launch
    # computes the rest through its fallback
    "chunks_two_segments_early_cut": dict(recurrent_max_len=-2, variant=4),
    "chunks_t_form": dict(recurrent_max_len=-2, variant=1),
    "token": dict(recurrent_max_len=1 << 30, recurrent_variant=0),
    "block": dict(recurrent_max_len=1 << 30, recurrent_variant=10),
}


def _inputs(T, cu, seed):
    inp = O.make_prefill_inputs([T], seed=seed, with_state=False)
    N = len(cu) - 1
    rng = np.random.default_rng(seed + 1000)
    inp["state"] = (0.05 * rng.standard_normal((N, 8, 128, 128))).astype(np.float32)
    inp["cu_seqlens"] = np.asarray(cu, dtype=np.int64)
    return inp


def _to_dev(inp, dev):
    bf = torch.bfloat16
    d = {n: torch.from_numpy(np.ascontiguousarray(inp[n])).to(dev).to(bf)
         for n in ("q", "k", "v", "a", "b")}
    for n in ("A_log", "dt_bias", "state", "cu_seqlens"):
        d[n] = torch.from_numpy(inp[n]).to(dev)
    return d


def _uncovered(T, cu):
    rows = np.ones(T, dtype=bool)
    rows[cu[0]:cu[-1]] = False
    return rows


def _call(d, out, ns, scale, **kw):
    prefill.kernel(d["q"], d["k"], d["v"], d["state"], d["A_log"], d["a"], d["dt_bias"], d["b"],
                   d["cu_seqlens"], scale, out, ns, **kw)


@pytest.mark.parametrize("route", list(ROUTES))
@pytest.mark.parametrize("T,cu", CASES)
def test_partial_cu_seqlens_matches_reference(cuda_device, T, cu, route):
    dev = cuda_device
    kw = ROUTES[route]
    N = len(cu) - 1
    if route.startswith("chunks_") and N != 1:
        pytest.skip("the explicit one-sequence variants apply to N = 1")
    if route in ("token", "block") and T > 1000:
        pytest.skip("long single sequences go through the chunks")
    print(f"partial cu T={T} cu={cu} route={route}", flush=True)
    inp = _inputs(T, cu, seed=T + 7 * N)
    d = _to_dev(inp, dev)
    out = torch.full((T, 8, 128), 3.0, dtype=torch.bfloat16, device=dev)
    ns = torch.full((N, 8, 128, 128), 5.0, dtype=torch.float32, device=dev)
    _call(d, out, ns, inp["scale"], **kw)
    torch.cuda.synchronize()
    o = out.float().cpu().numpy()
    o_ref, s_ref = O.prefill_seq_c(**inp)
    assert not o[_uncovered(T, cu)].any(), "rows outside [cu[0], cu[N]) must be zero"
    assert_output_close(o, o_ref)
    assert_state_close(ns.cpu().numpy(), s_ref)


def test_no_sequences_zeroes_the_output(cuda_device):
    dev = cuda_device
    T = 200
    inp = _inputs(T, [37], seed=3)
    d = _to_dev(inp, dev)
    out = torch.full((T, 8, 128), 3.0, dtype=torch.bfloat16, device=dev)
    ns = torch.empty((0, 8, 128, 128), dtype=torch.float32, device=dev)
    _call(d, out, ns, inp["scale"])
    torch.cuda.synchronize()
    assert not out.float().cpu().numpy().any()


def test_misaligned_output_view(cuda_device):
    # a contiguous output view 2 bytes into its storage: computed into an
    # aligned buffer and copied, as the reference copies its result
    dev = cuda_device
    T, cu = 300, [7, 7, 150, 290]
    inp = _inputs(T, cu, seed=11)
    d = _to_dev(inp, dev)
    store = torch.full((T * 8 * 128 + 1,), 3.0, dtype=torch.bfloat16, device=dev)
    out = store[1:].view(T, 8, 128)
    assert out.data_ptr() % 16
    ns = torch.empty((3, 8, 128, 128), dtype=torch.float32, device=dev)
    _call(d, out, ns, inp["scale"])
    torch.cuda.synchronize()
    o_ref, s_ref = O.prefill_seq_c(**inp)
    assert_output_close(out.float().cpu().numpy(), o_ref)
    assert_state_close(ns.cpu().numpy(), s_ref)
    assert float(store[0]) == 3.0


# One captured graph per T, replayed with cu_seqlens contents that cover the
# buffer, pad it, or start late; every replay equals the eager call.
GRAPH_REPLAYS = {
    (1, 2500): [[0, 2500], [0, 2100], [300, 1900], [0, 2500]],
    (2, 600): [[0, 300, 600], [0, 100, 200], [50, 50, 500], [0, 300, 600]],
}


@pytest.mark.parametrize("N,T", list(GRAPH_REPLAYS))
def test_graph_replays_follow_partial_cu_seqlens(cuda_device, N, T):
    dev = cuda_device
    replays = GRAPH_REPLAYS[(N, T)]
    print(f"partial cu graph N={N} T={T}", flush=True)
    inp = _inputs(T, replays[0], seed=70)
    d = _to_dev(inp, dev)
    scale = float(inp["scale"])
    ws = prefill.alloc_workspace(T, N, dev)
    out = torch.empty((T, 8, 128), dtype=torch.bfloat16, device=dev)
    ns = torch.empty((N, 8, 128, 128), dtype=torch.float32, device=dev)

    side = torch.cuda.Stream(device=dev)
    side.wait_stream(torch.cuda.current_stream(dev))
    with torch.cuda.stream(side):
        _call(d, out, ns, scale, workspace=ws)
    torch.cuda.current_stream(dev).wait_stream(side)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        _call(d, out, ns, scale, workspace=ws)
    torch.cuda.synchronize()

    for rep, cu in enumerate(replays[1:]):
        print(f"  replay {rep} cu={cu}", flush=True)
        inp = _inputs(T, cu, seed=71 + rep)
        for n, t in _to_dev(inp, dev).items():
            d[n].copy_(t)
        g.replay()
        torch.cuda.synchronize()
        o_g, s_g = out.clone(), ns.clone()
        o_e = torch.full_like(out, 3.0)
        s_e = torch.empty_like(ns)
        _call(d, o_e, s_e, scale, workspace=ws)
        torch.cuda.synchronize()
        assert torch.equal(o_g, o_e), f"replay {rep}: output differs from the eager call"
        assert torch.equal(s_g, s_e), f"replay {rep}: state differs from the eager call"
        o_ref, s_ref = O.prefill_seq_c(**inp)
        o = o_g.float().cpu().numpy()
        assert not o[_uncovered(T, cu)].any()
        assert_output_close(o, o_ref)
        assert_state_close(s_g.cpu().numpy(), s_ref)
