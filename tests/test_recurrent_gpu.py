"""The token-sequential kernel on the GPU: prefill of batches of short
sequences (the path chosen from the longest sequence, on the host when T
decides it, else on the device), the path choice itself, and multi-token
decode (T > 1).

Oracle: the sequential recurrence of reference/gdn_prefill_ref.py:71-89
(oracle/gdn_seq.c through O.prefill_seq_c, pinned in tests/test_oracle.py).
Tolerance as everywhere (conftest.py): bf16 output atol = rtol = 1e-2; f32
state atol = 1e-3 * max|state_ref|.  The token-sequential kernel computes in
f32 in the reference's order, so its state is also held to 1e-5 * max|ref|.
"""

import math

import numpy as np
import pytest
import torch

from conftest import assert_output_close, assert_state_close
from oracle import gdn_oracle as O

pytestmark = pytest.mark.gpu

from gdn_amd import decode, prefill  # noqa: E402


def _to_dev(inp, dev, cu_dtype=torch.int64):
    bf = torch.bfloat16
    d = {n: torch.from_numpy(np.ascontiguousarray(inp[n])).to(dev).to(bf)
         for n in ("q", "k", "v", "a", "b")}
    for n in ("A_log", "dt_bias"):
        d[n] = torch.from_numpy(inp[n]).to(dev)
    d["state"] = None if inp["state"] is None else torch.from_numpy(inp["state"]).to(dev)
    if "cu_seqlens" in inp:
        d["cu_seqlens"] = torch.from_numpy(inp["cu_seqlens"]).to(dev).to(cu_dtype)
    d["scale"] = inp["scale"]
    return d


def _prefill(d, dev, in_place=False, **kw):
    T = d["q"].shape[0]
    N = d["cu_seqlens"].numel() - 1
    out = torch.empty((T, 8, 128), dtype=torch.bfloat16, device=dev)
    ns = d["state"] if in_place else torch.empty((N, 8, 128, 128), dtype=torch.float32,
                                                 device=dev)
    prefill.kernel(d["q"], d["k"], d["v"], d["state"], d["A_log"], d["a"], d["dt_bias"],
                   d["b"], d["cu_seqlens"], d["scale"], out, ns, **kw)
    torch.cuda.synchronize()
    return out, ns


def _check(out, ns, inp, tight=False):
    o_ref, s_ref = O.prefill_seq_c(**inp)
    o = out.float().cpu().numpy()
    s = ns.cpu().numpy()
    assert_output_close(o, o_ref)
    assert_state_close(s, s_ref)
    if tight:
        assert_state_close(s, s_ref, rel_atol=1e-5, what="state (f32 sequential bound)")


# The whole call through the token-sequential kernel (routing length above T).
ALL_SEQUENTIAL = 1 << 30

SHORT_CASES = [
    ([1], True), ([2], False), ([16], True), ([63], True), ([64], False), ([65], True),
    ([200], True), ([256], True), ([6, 49, 61], True), ([0, 5, 0, 100], True), ([0], True),
    ([1] * 40, True), ([3, 0, 7, 250], False),
]


@pytest.mark.parametrize("lens, with_state", SHORT_CASES)
def test_short_prefill_matches_oracle(cuda_device, lens, with_state):
    print(f"short prefill lens={lens if len(lens) < 8 else f'{len(lens)}x{lens[0]}'} "
          f"state={with_state}", flush=True)
    inp = O.make_prefill_inputs(lens, seed=7 + len(lens), with_state=with_state)
    out, ns = _prefill(_to_dev(inp, cuda_device), cuda_device, recurrent_max_len=ALL_SEQUENTIAL)
    _check(out, ns, inp, tight=True)


def test_short_prefill_int32_cu_and_in_place(cuda_device):
    lens = [6, 49, 0, 61]
    inp = O.make_prefill_inputs(lens, seed=12)
    d = _to_dev(inp, cuda_device, cu_dtype=torch.int32)
    out, ns = _prefill(d, cuda_device, in_place=True, recurrent_max_len=ALL_SEQUENTIAL)
    assert ns.data_ptr() == d["state"].data_ptr()
    _check(out, ns, inp, tight=True)


# configs[3] lengths under several path lengths: chunked (-1 = built-in, 64,
# 300, -2 = never sequential, 0), token by token decided on the device (4096:
# longest 2040 <= 4096 < T) and on the host (ALL_SEQUENTIAL >= T).
@pytest.mark.parametrize("rec_max", [-1, 64, 300, -2, 4096, 0, ALL_SEQUENTIAL])
def test_path_choice_on_configs3(cuda_device, rec_max):
    lens = [6, 49, 294, 1800, 2040, 61]
    print(f"routing rec_max={rec_max}", flush=True)
    inp = O.make_prefill_inputs(lens, seed=3)
    out, ns = _prefill(_to_dev(inp, cuda_device), cuda_device, recurrent_max_len=rec_max)
    _check(out, ns, inp)


def test_routing_zero_length_sequences_get_zero_state(cuda_device):
    lens = [0, 300, 0, 20, 0]
    inp = O.make_prefill_inputs(lens, seed=13)
    for rec_max in (-2, -1, 0, 64, 310):  # 310: sequential, decided on the device
        out, ns = _prefill(_to_dev(inp, cuda_device), cuda_device, recurrent_max_len=rec_max)
        s = ns.cpu().numpy()
        assert not s[[0, 2, 4]].any(), f"rec_max={rec_max}"
        _check(out, ns, inp)


def _cost_by_token(L, T, hv, g):
    return 3.56 + 0.216 * L + 0.00297 * T * hv + 0.0131 * g


def _cost_by_block(L, g):
    per_block = 2.8 if g <= 128 else 3.5 if g <= 256 else 4.7
    return (4.5 + 0.015 * g + 0.008 * max(g - 256, 0)
            + math.ceil(g / 512) * math.ceil(L / 16) * per_block)


def _t_form_wins(nt, lc, units):
    large = nt >= 144 and (nt > 3 * lc or (nt >= 384 and nt >= 1.5 * lc))
    small = units <= 768 and lc <= 12 and nt > lc
    return large or small


def _cost_by_chunks_form(L, nt, hv, N, t):
    lc, units = math.ceil(L / 64), N * hv * 8
    steps = max(lc, nt * hv / 64)
    if t:
        return 20.6 + 0.0457 * nt * hv + (0.631 if units <= 256 else 0.785) * steps
    return 19.8 + 0.0567 * nt * hv + (0.373 if units <= 256 else 0.454) * steps


def _cost_by_chunks(L, nt, hv, N):
    return _cost_by_chunks_form(L, nt, hv, N, _t_form_wins(nt, math.ceil(L / 64), N * hv * 8))


def _expected_path(lens, hv=8):
    """The built-in path choice of gdn_prefill_fwd (gdn_prefill.hip, cost
    models of gdn_host.h), restated: "token", "block" or "chunks"."""
    T, N, L = sum(lens), len(lens), max(lens)
    if T <= 96:
        if N == 1 and _cost_by_block(T, hv) < _cost_by_token(T, T, hv, hv):
            return "block"
        return "token"
    if N == 1:
        return "chunks"
    g, mean = N * hv, math.ceil(T / N)
    by_token, by_block = _cost_by_token(mean, T, hv, g), _cost_by_block(mean, g)
    kind = "block" if by_block < by_token else "token"
    if min(by_token, by_block) + 9 >= _cost_by_chunks(mean, N * math.ceil(mean / 64), hv, N):
        return "chunks"  # decided on the host
    nt = sum(math.ceil(n / 64) for n in lens)
    seq = _cost_by_block(L, g) if kind == "block" else _cost_by_token(L, T, hv, g)
    return kind if seq + 4 <= _cost_by_chunks(L, nt, hv, N) else "chunks"


def _expected_multi_kind(B, T, hv=8):
    """The built-in kernel of gdn_decode_multi_fwd for T > 1 tokens per row."""
    g = B * hv
    return "block" if _cost_by_block(T, g) < _cost_by_token(T, B * T, hv, g) else "token"


def _path_flag(dev, T, N):
    """The path flag the index kernel leaves in the per-stream workspace."""
    ws = prefill._workspace(dev, torch.cuda.current_stream(dev).cuda_stream, 0)
    chunks_bytes = (O.max_chunks(T, N) * 16 + 255) // 256 * 256
    flag_at = chunks_bytes + (N + 1) * 4
    return int(ws[flag_at:flag_at + 4].cpu().numpy().view(np.int32)[0])


def _lens_1500():
    lens = np.random.default_rng(5).integers(0, 4, 1500).tolist()
    lens[3] = 70
    return lens


# Batches of T > 96 tokens in N > 1 sequences (the host settles the clear
# cases, the device the rest), with the path the cost models pick: token by
# token, 16-token blocks or chunks.
DEVICE_CHOICE = {
    "256x1": ([1] * 256, "token"),
    "64x16": ([16] * 64, "block"),
    "mixed40": ([3, 17, 80, 0, 40] * 8, "block"),
    "1500": (_lens_1500(), "token"),
    "10x2+200": ([2] * 10 + [200], "chunks"),
    "16x8": ([8] * 16, "block"),
    "32x128": ([128] * 32, "block"),
    "3x40+300": ([40] * 3 + [300], "chunks"),
}


@pytest.mark.parametrize("name", list(DEVICE_CHOICE))
def test_device_path_choice(cuda_device, name):
    lens, want = DEVICE_CHOICE[name]
    T, N = sum(lens), len(lens)
    assert _expected_path(lens) == want
    print(f"device path choice {name}: T={T} N={N} path={want}", flush=True)
    inp = O.make_prefill_inputs(lens, seed=15)
    out, ns = _prefill(_to_dev(inp, cuda_device), cuda_device)
    assert _path_flag(cuda_device, T, N) == int(want != "chunks")
    _check(out, ns, inp, tight=want == "token")


def test_recurrent_tilings_are_identical(cuda_device):
    lens = [6, 49, 200, 1]
    inp = O.make_prefill_inputs(lens, seed=14)
    d = _to_dev(inp, cuda_device)
    ref_o, ref_s = _prefill(d, cuda_device, recurrent_variant=0, recurrent_max_len=ALL_SEQUENTIAL)
    _check(ref_o, ref_s, inp, tight=True)
    for var in range(1, 10):
        o, s = _prefill(d, cuda_device, recurrent_variant=var, recurrent_max_len=ALL_SEQUENTIAL)
        assert torch.equal(o, ref_o), f"tiling {var}: output differs"
        assert torch.equal(s, ref_s), f"tiling {var}: state differs"


# ---------------------------------------------------------------------------
# multi-token decode
# ---------------------------------------------------------------------------

def _multi_inputs(B, T, seed, with_state=True):
    """[B, T, ...] decode inputs and the same data as a packed prefill batch
    of B sequences of T tokens (the oracle's form)."""
    inp = O.make_prefill_inputs([T] * B, seed=seed, with_state=with_state)
    dec = dict(inp)
    for n, tail in (("q", (4, 128)), ("k", (4, 128)), ("v", (8, 128)), ("a", (8,)),
                    ("b", (8,))):
        dec[n] = inp[n].reshape((B, T) + tail)
    del dec["cu_seqlens"]
    return inp, dec


def _decode_multi(d, B, T, dev, in_place=False, variant=-1):
    out = torch.empty((B, T, 8, 128), dtype=torch.bfloat16, device=dev)
    ns = d["state"] if in_place else torch.empty((B, 8, 128, 128), dtype=torch.float32,
                                                 device=dev)
    decode.kernel(d["q"], d["k"], d["v"], d["state"], d["A_log"], d["a"], d["dt_bias"], d["b"],
                  d["scale"], out, ns, variant=variant)
    torch.cuda.synchronize()
    return out, ns


@pytest.mark.parametrize("B, T", [(1, 2), (3, 5), (16, 4), (64, 2), (64, 8), (32, 16)])
def test_multi_token_decode_matches_oracle(cuda_device, B, T):
    print(f"multi-token decode B={B} T={T}", flush=True)
    inp, dec = _multi_inputs(B, T, seed=20 + B + T)
    out, ns = _decode_multi(_to_dev(dec, cuda_device), B, T, cuda_device)
    _check(out.reshape(B * T, 8, 128), ns, inp, tight=_expected_multi_kind(B, T) == "token")


def test_multi_token_decode_equals_successive_steps(cuda_device):
    B, T = 8, 4
    inp, dec = _multi_inputs(B, T, seed=31)
    d = _to_dev(dec, cuda_device)
    out, ns = _decode_multi(d, B, T, cuda_device)
    state = d["state"].clone()
    for t in range(T):
        o1 = torch.empty((B, 1, 8, 128), dtype=torch.bfloat16, device=cuda_device)
        s1 = torch.empty_like(state)
        sl = slice(t, t + 1)
        decode.kernel(d["q"][:, sl].contiguous(), d["k"][:, sl].contiguous(),
                      d["v"][:, sl].contiguous(), state, d["A_log"], d["a"][:, sl].contiguous(),
                      d["dt_bias"], d["b"][:, sl].contiguous(), d["scale"], o1, s1)
        assert_output_close(out[:, sl].float().cpu().numpy(), o1.float().cpu().numpy(),
                            atol=1e-2, rtol=1e-2, what=f"token {t}")
        state = s1
    torch.cuda.synchronize()
    assert_state_close(ns.cpu().numpy(), state.cpu().numpy(), rel_atol=1e-5)


def test_multi_token_decode_in_place_and_no_state(cuda_device):
    B, T = 4, 3
    inp, dec = _multi_inputs(B, T, seed=32)
    d = _to_dev(dec, cuda_device)
    out, ns = _decode_multi(d, B, T, cuda_device, in_place=True)
    assert ns.data_ptr() == d["state"].data_ptr()
    _check(out.reshape(B * T, 8, 128), ns, inp, tight=True)
    inp0, dec0 = _multi_inputs(B, T, seed=33, with_state=False)
    out0, ns0 = _decode_multi(_to_dev(dec0, cuda_device), B, T, cuda_device)
    _check(out0.reshape(B * T, 8, 128), ns0, inp0, tight=True)


def test_multi_token_decode_tilings_are_identical(cuda_device):
    B, T = 5, 3
    inp, dec = _multi_inputs(B, T, seed=34)
    d = _to_dev(dec, cuda_device)
    ref_o, ref_s = _decode_multi(d, B, T, cuda_device, variant=0)
    for var in range(1, 10):
        o, s = _decode_multi(d, B, T, cuda_device, variant=var)
        assert torch.equal(o, ref_o) and torch.equal(s, ref_s), f"tiling {var}"
    _check(ref_o.reshape(B * T, 8, 128), ref_s, inp, tight=True)


# ---------------------------------------------------------------------------
# the 16-token block kernel (gdn_block.hip; recurrent variant BLOCK)
# ---------------------------------------------------------------------------

BLOCK = 10


def _state_err(ns, inp):
    _, s_ref = O.prefill_seq_c(**inp)
    s = ns.cpu().numpy()
    return float(np.abs(s - s_ref).max() / max(np.abs(s_ref).max(), 1e-30))


@pytest.mark.parametrize("lens, with_state", SHORT_CASES + [([17, 31, 32, 33], True)])
def test_block_kernel_short_prefill_matches_oracle(cuda_device, lens, with_state):
    print(f"block kernel prefill lens={lens} state={with_state}", flush=True)
    inp = O.make_prefill_inputs(lens, seed=60 + len(lens), with_state=with_state)
    out, ns = _prefill(_to_dev(inp, cuda_device), cuda_device, recurrent_max_len=ALL_SEQUENTIAL,
                       recurrent_variant=BLOCK)
    print(f"  state error {_state_err(ns, inp):.2e} of max|S|", flush=True)
    _check(out, ns, inp)


@pytest.mark.parametrize("B, T", [(1, 2), (3, 5), (16, 4), (64, 8), (4, 33), (2, 16), (2, 17)])
def test_block_kernel_multi_token_decode(cuda_device, B, T):
    print(f"block kernel multi-token decode B={B} T={T}", flush=True)
    inp, dec = _multi_inputs(B, T, seed=70 + B + T)
    out, ns = _decode_multi(_to_dev(dec, cuda_device), B, T, cuda_device, variant=BLOCK)
    print(f"  state error {_state_err(ns, inp):.2e} of max|S|", flush=True)
    _check(out.reshape(B * T, 8, 128), ns, inp)


def test_block_kernel_extreme_gates_in_place_and_no_state(cuda_device):
    # Gates around softplus' threshold, beta saturated at 0 and 1, near-unit
    # and underflowing decays (as the chunk pipeline's extreme-gate test).
    lens = [40, 16, 100]
    inp = O.make_prefill_inputs(lens, seed=71)
    rng = np.random.default_rng(71)
    T = sum(lens)
    a_h = np.array([30.0, -30.0, 20.0, 0.0, 19.5, -5.0, 5.0, 1.0], np.float32)
    b_h = np.array([-40.0, 40.0, 0.0, 8.0, -8.0, 1.0, -1.0, 0.0], np.float32)
    inp["a"][:] = O.bf16_round(a_h[None, :] + rng.normal(0, 0.5, (T, 8)).astype(np.float32))
    inp["b"][:] = O.bf16_round(b_h[None, :] + rng.normal(0, 0.5, (T, 8)).astype(np.float32))
    inp["A_log"][:] = np.array([-10.0, 2.7, 0.0, -20.0, 1.0, 0.5, 0.1, 2.0], np.float32)
    print("block kernel extreme gates", flush=True)
    d = _to_dev(inp, cuda_device)
    out, ns = _prefill(d, cuda_device, recurrent_max_len=ALL_SEQUENTIAL, recurrent_variant=BLOCK)
    assert torch.isfinite(out.float()).all() and torch.isfinite(ns).all()
    _check(out, ns, inp)
    oi, si = _prefill(d, cuda_device, in_place=True, recurrent_max_len=ALL_SEQUENTIAL,
                      recurrent_variant=BLOCK)
    assert torch.equal(oi, out) and torch.equal(si, ns)
    inp["state"] = None
    o0, s0 = _prefill(_to_dev(inp, cuda_device), cuda_device, recurrent_max_len=ALL_SEQUENTIAL,
                      recurrent_variant=BLOCK)
    _check(o0, s0, inp)
