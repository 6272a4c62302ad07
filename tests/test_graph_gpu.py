"""HIP-graph capture of both entry points: the allocation-free serving path.

A graph is captured once with torch.cuda.graph around the DPS ``kernel``
and replayed several times; between replays the program writes new inputs
into the captured tensors (for prefill also new ``cu_seqlens`` contents with
the same T and N, which the device-built chunk index must pick up), runs the
same call eagerly and synchronises.  Every replay must equal the eager result
bit for bit (same kernels, same inputs) and the oracle within the parity
tolerance.  The reference could not capture its prefill at all
(OPTIMIZATION_LOG.md:150-153: Triton dispatch and a D2H ``.tolist()``), and
its identity-keyed chunk cache goes stale when cu_seqlens changes in place
(fla_kernels.py:959-972).

Also the clone mode of FlashInfer-Bench (every argument freshly allocated per
call, OPTIMIZATION_LOG.md:263-300): results stay identical and the library
allocates nothing after the first call on a stream.
"""

import numpy as np
import pytest
import torch

from conftest import assert_output_close, assert_state_close
from oracle import gdn_oracle as O

pytestmark = pytest.mark.gpu

from gdn_amd import decode, prefill  # noqa: E402


def _dev(x, dev, dtype):
    return torch.from_numpy(np.ascontiguousarray(x)).to(dev).to(dtype)


def _fill_decode(static, inp):
    bf = torch.bfloat16
    for n in ("q", "k", "v", "a", "b"):
        static[n].copy_(_dev(inp[n], static[n].device, bf))
    for n in ("A_log", "dt_bias", "state"):
        static[n].copy_(torch.from_numpy(inp[n]))


def test_decode_graph_replays_match_eager(cuda_device):
    dev, B = cuda_device, 16
    print(f"decode graph B={B}", flush=True)
    inp = O.make_decode_inputs(B, seed=21)
    st = {n: _dev(inp[n], dev, torch.bfloat16) for n in ("q", "k", "v", "a", "b")}
    for n in ("A_log", "dt_bias", "state"):
        st[n] = torch.from_numpy(inp[n]).to(dev)
    out = torch.empty((B, 1, 8, 128), dtype=torch.bfloat16, device=dev)
    ns = torch.empty((B, 8, 128, 128), dtype=torch.float32, device=dev)
    scale = float(inp["scale"])

    def call(o, s):
        decode.kernel(st["q"], st["k"], st["v"], st["state"], st["A_log"], st["a"],
                      st["dt_bias"], st["b"], scale, o, s)

    side = torch.cuda.Stream(device=dev)
    side.wait_stream(torch.cuda.current_stream(dev))
    with torch.cuda.stream(side):
        call(out, ns)
    torch.cuda.current_stream(dev).wait_stream(side)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        call(out, ns)
    torch.cuda.synchronize()

    for rep in range(3):
        inp = O.make_decode_inputs(B, seed=100 + rep)
        _fill_decode(st, inp)
        g.replay()
        torch.cuda.synchronize()
        o_g, s_g = out.clone(), ns.clone()
        o_e = torch.empty_like(out)
        s_e = torch.empty_like(ns)
        call(o_e, s_e)
        torch.cuda.synchronize()
        assert torch.equal(o_g, o_e), f"replay {rep}: output differs from the eager call"
        assert torch.equal(s_g, s_e), f"replay {rep}: state differs from the eager call"
        o_ref, s_ref = O.decode(**inp)
        assert_output_close(o_g.float().cpu().numpy(), o_ref)
        assert_state_close(s_g.cpu().numpy(), s_ref)


def _prefill_static(T, N, dev):
    bf = torch.bfloat16
    return {
        "q": torch.empty((T, 4, 128), dtype=bf, device=dev),
        "k": torch.empty((T, 4, 128), dtype=bf, device=dev),
        "v": torch.empty((T, 8, 128), dtype=bf, device=dev),
        "a": torch.empty((T, 8), dtype=bf, device=dev),
        "b": torch.empty((T, 8), dtype=bf, device=dev),
        "A_log": torch.empty(8, dtype=torch.float32, device=dev),
        "dt_bias": torch.empty(8, dtype=torch.float32, device=dev),
        "state": torch.empty((N, 8, 128, 128), dtype=torch.float32, device=dev),
        "cu_seqlens": torch.empty(N + 1, dtype=torch.int64, device=dev),
    }


def _fill_prefill(st, inp):
    for n in ("q", "k", "v", "a", "b"):
        st[n].copy_(_dev(inp[n], st[n].device, torch.bfloat16))
    for n in ("A_log", "dt_bias", "state", "cu_seqlens"):
        st[n].copy_(torch.from_numpy(inp[n]))


# Same T = 300 and N = 3 for every replay; only the split into sequences
# changes (including zero-length and single-token sequences).
REPLAY_LENS = [[100, 100, 100], [0, 37, 263], [299, 1, 0], [64, 172, 64]]


def test_prefill_graph_replays_follow_new_cu_seqlens(cuda_device):
    dev = cuda_device
    T, N = sum(REPLAY_LENS[0]), len(REPLAY_LENS[0])
    print(f"prefill graph T={T} N={N}", flush=True)
    st = _prefill_static(T, N, dev)
    inp = O.make_prefill_inputs(REPLAY_LENS[0], seed=31)
    _fill_prefill(st, inp)
    scale = float(inp["scale"])
    ws = prefill.alloc_workspace(T, N, dev)
    out = torch.empty((T, 8, 128), dtype=torch.bfloat16, device=dev)
    ns = torch.empty((N, 8, 128, 128), dtype=torch.float32, device=dev)

    def call(o, s):
        prefill.kernel(st["q"], st["k"], st["v"], st["state"], st["A_log"], st["a"],
                       st["dt_bias"], st["b"], st["cu_seqlens"], scale, o, s, workspace=ws)

    side = torch.cuda.Stream(device=dev)
    side.wait_stream(torch.cuda.current_stream(dev))
    with torch.cuda.stream(side):
        call(out, ns)
    torch.cuda.current_stream(dev).wait_stream(side)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        call(out, ns)
    torch.cuda.synchronize()

    for rep, lens in enumerate(REPLAY_LENS[1:] + REPLAY_LENS[:1]):
        print(f"  replay {rep} lens={lens}", flush=True)
        inp = O.make_prefill_inputs(lens, seed=40 + rep)
        _fill_prefill(st, inp)
        g.replay()
        torch.cuda.synchronize()
        o_g, s_g = out.clone(), ns.clone()
        o_e = torch.empty_like(out)
        s_e = torch.empty_like(ns)
        call(o_e, s_e)
        torch.cuda.synchronize()
        assert torch.equal(o_g, o_e), f"replay {rep}: output differs from the eager call"
        assert torch.equal(s_g, s_e), f"replay {rep}: state differs from the eager call"
        o_ref, s_ref = O.prefill_seq_c(**inp)
        assert_output_close(o_g.float().cpu().numpy(), o_ref)
        assert_state_close(s_g.cpu().numpy(), s_ref)


def test_prefill_clone_mode_allocates_nothing_after_first_call(cuda_device):
    dev = cuda_device
    lens = [6, 49, 294, 61]
    inp = O.make_prefill_inputs(lens, seed=3)
    T, N = sum(lens), len(lens)
    base = _prefill_static(T, N, dev)
    _fill_prefill(base, inp)
    scale = float(inp["scale"])

    def fresh_call():
        a = {n: t.clone() for n, t in base.items()}
        o = torch.empty((T, 8, 128), dtype=torch.bfloat16, device=dev)
        s = torch.empty((N, 8, 128, 128), dtype=torch.float32, device=dev)
        prefill.kernel(a["q"], a["k"], a["v"], a["state"], a["A_log"], a["a"], a["dt_bias"],
                       a["b"], a["cu_seqlens"], scale, o, s)
        return o, s

    o0, s0 = fresh_call()
    torch.cuda.synchronize()
    before = torch.cuda.memory_allocated(dev)
    for _ in range(3):
        o, s = fresh_call()
        torch.cuda.synchronize()
        assert torch.equal(o, o0) and torch.equal(s, s0)
        del o, s
    torch.cuda.synchronize()
    assert torch.cuda.memory_allocated(dev) == before
    o_ref, s_ref = O.prefill_seq_c(**inp)
    assert_output_close(o0.float().cpu().numpy(), o_ref)
    assert_state_close(s0.cpu().numpy(), s_ref)


def test_prefill_workspace_argument_checks(cuda_device):
    dev = cuda_device
    inp = O.make_prefill_inputs([70], seed=5)
    st = _prefill_static(70, 1, dev)
    _fill_prefill(st, inp)
    out = torch.empty((70, 8, 128), dtype=torch.bfloat16, device=dev)
    ns = torch.empty((1, 8, 128, 128), dtype=torch.float32, device=dev)
    args = (st["q"], st["k"], st["v"], st["state"], st["A_log"], st["a"], st["dt_bias"], st["b"],
            st["cu_seqlens"], None, out, ns)
    small = torch.empty(prefill.workspace_bytes(70, 1) - 256, dtype=torch.uint8, device=dev)
    with pytest.raises(Exception, match="workspace"):
        prefill.kernel(*args, workspace=small)
    with pytest.raises(ValueError, match="uint8"):
        prefill.kernel(*args, workspace=torch.empty(1 << 20, dtype=torch.float32, device=dev))
    ws = prefill.alloc_workspace(70, 1, dev)
    prefill.kernel(*args, workspace=ws)
    torch.cuda.synchronize()
    o_ref, s_ref = O.prefill_seq_c(**inp)
    assert_output_close(out.float().cpu().numpy(), o_ref)
    assert_state_close(ns.cpu().numpy(), s_ref)


def test_prefill_release_workspaces(cuda_device):
    # a call on a fresh stream caches a workspace for it; release_workspaces
    # hands it back (it was never captured), and the next call allocates anew
    # and gives the same result
    dev = cuda_device
    inp = O.make_prefill_inputs([300], seed=6)
    st = _prefill_static(300, 1, dev)
    _fill_prefill(st, inp)
    side = torch.cuda.Stream(device=dev)
    outs = []
    for _ in range(2):
        out = torch.empty((300, 8, 128), dtype=torch.bfloat16, device=dev)
        ns = torch.empty((1, 8, 128, 128), dtype=torch.float32, device=dev)
        side.wait_stream(torch.cuda.current_stream(dev))
        with torch.cuda.stream(side):
            prefill.kernel(st["q"], st["k"], st["v"], st["state"], st["A_log"], st["a"],
                           st["dt_bias"], st["b"], st["cu_seqlens"], None, out, ns)
        torch.cuda.synchronize()
        outs.append((out, ns))
        key = (dev.index, side.cuda_stream)
        assert key in prefill._workspaces
        assert prefill.release_workspaces() >= prefill.workspace_bytes(300, 1)
        assert key not in prefill._workspaces
    assert torch.equal(outs[0][0], outs[1][0]) and torch.equal(outs[0][1], outs[1][1])
    o_ref, s_ref = O.prefill_seq_c(**inp)
    assert_output_close(outs[0][0].float().cpu().numpy(), o_ref)
    assert_state_close(outs[0][1].cpu().numpy(), s_ref)


@pytest.mark.parametrize("T", [2500, 4500])
def test_prefill_graph_replays_two_segment_scan(cuda_device, T):
    # One sequence of 2500 tokens (40 chunks: the two-segment scan, its
    # second-segment output kernel and the new_state tiles), or of 4500 (71
    # chunks: the state launch also computes the first 21 chunks' output,
    # with progress words the intra launch zeroes), captured once and
    # replayed with new inputs; every replay equals the eager call.
    dev = cuda_device
    N = 1
    print(f"prefill graph two-segment T={T}", flush=True)
    st = _prefill_static(T, N, dev)
    inp = O.make_prefill_inputs([T], seed=50)
    _fill_prefill(st, inp)
    scale = float(inp["scale"])
    ws = prefill.alloc_workspace(T, N, dev)
    out = torch.empty((T, 8, 128), dtype=torch.bfloat16, device=dev)
    ns = torch.empty((N, 8, 128, 128), dtype=torch.float32, device=dev)

    def call(o, s):
        prefill.kernel(st["q"], st["k"], st["v"], st["state"], st["A_log"], st["a"],
                       st["dt_bias"], st["b"], st["cu_seqlens"], scale, o, s, workspace=ws)

    side = torch.cuda.Stream(device=dev)
    side.wait_stream(torch.cuda.current_stream(dev))
    with torch.cuda.stream(side):
        call(out, ns)
    torch.cuda.current_stream(dev).wait_stream(side)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        call(out, ns)
    torch.cuda.synchronize()

    for rep in range(3):
        print(f"  replay {rep}", flush=True)
        inp = O.make_prefill_inputs([T], seed=51 + rep, slow_decay_heads=(7,) if rep else ())
        _fill_prefill(st, inp)
        g.replay()
        torch.cuda.synchronize()
        o_g, s_g = out.clone(), ns.clone()
        o_e = torch.empty_like(out)
        s_e = torch.empty_like(ns)
        call(o_e, s_e)
        torch.cuda.synchronize()
        assert torch.equal(o_g, o_e), f"replay {rep}: output differs from the eager call"
        assert torch.equal(s_g, s_e), f"replay {rep}: state differs from the eager call"
        o_ref, s_ref = O.prefill_seq_c(**inp)
        assert_output_close(o_g.float().cpu().numpy(), o_ref)
        assert_state_close(s_g.cpu().numpy(), s_ref)


# Same T = 1024 and N = 64 for every replay; the device picks the path per
# replay from the new cu_seqlens: 16-token blocks or the chunks.
PATH_REPLAYS = [
    ([16] * 64, 1),
    ([1000] + [0] * 62 + [24], 0),
    ([15] * 63 + [79], 1),
    ([0] * 63 + [1024], 0),
]


def test_prefill_graph_replays_follow_the_device_path_choice(cuda_device):
    dev = cuda_device
    T, N = 1024, 64
    print(f"prefill graph device path choice T={T} N={N}", flush=True)
    st = _prefill_static(T, N, dev)
    inp = O.make_prefill_inputs(PATH_REPLAYS[0][0], seed=60)
    _fill_prefill(st, inp)
    scale = float(inp["scale"])
    ws = prefill.alloc_workspace(T, N, dev)
    flag_at = (O.max_chunks(T, N) * 16 + 255) // 256 * 256 + (N + 1) * 4
    out = torch.empty((T, 8, 128), dtype=torch.bfloat16, device=dev)
    ns = torch.empty((N, 8, 128, 128), dtype=torch.float32, device=dev)

    def call(o, s):
        prefill.kernel(st["q"], st["k"], st["v"], st["state"], st["A_log"], st["a"],
                       st["dt_bias"], st["b"], st["cu_seqlens"], scale, o, s, workspace=ws)

    side = torch.cuda.Stream(device=dev)
    side.wait_stream(torch.cuda.current_stream(dev))
    with torch.cuda.stream(side):
        call(out, ns)
    torch.cuda.current_stream(dev).wait_stream(side)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        call(out, ns)
    torch.cuda.synchronize()

    for rep, (lens, want_flag) in enumerate(PATH_REPLAYS[1:] + PATH_REPLAYS[:1]):
        print(f"  replay {rep} longest={max(lens)}", flush=True)
        inp = O.make_prefill_inputs(lens, seed=61 + rep)
        _fill_prefill(st, inp)
        g.replay()
        torch.cuda.synchronize()
        flag = int(ws[flag_at:flag_at + 4].cpu().numpy().view(np.int32)[0])
        assert flag == want_flag, f"replay {rep}: path flag {flag}"
        o_g, s_g = out.clone(), ns.clone()
        o_e = torch.empty_like(out)
        s_e = torch.empty_like(ns)
        call(o_e, s_e)
        torch.cuda.synchronize()
        assert torch.equal(o_g, o_e), f"replay {rep}: output differs from the eager call"
        assert torch.equal(s_g, s_e), f"replay {rep}: state differs from the eager call"
        o_ref, s_ref = O.prefill_seq_c(**inp)
        assert_output_close(o_g.float().cpu().numpy(), o_ref)
        assert_state_close(s_g.cpu().numpy(), s_ref)
