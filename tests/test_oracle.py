"""Pins the CPU oracle (oracle/gdn_oracle.py, oracle/gdn_seq.c).

The reference ships no golden vectors for this path, so every oracle function
is checked against what the mathematics fixes: closed forms, limits,
invariances, brute force and an independent algorithm (chunked WY form vs
the token-by-token recurrence).  Each check is chosen so that a plausible
slip -- a dropped term, a wrong sign, a transposed state, a wrong GVA head --
fails it.
"""

import math

import numpy as np
import pytest
import scipy.linalg

from oracle import gdn_oracle as O


def _rng(seed=0):
    return np.random.default_rng(seed)


# ---------------------------------------------------------------- bf16 helpers

def test_bf16_rounding_known_values():
    x = np.array([1.0, 1.0 + 2 ** -8, 1.0 + 2 ** -7 + 2 ** -8, 1.0 + 2 ** -9, -2.5,
                  np.inf, -np.inf, 3.0e38], np.float32)
    # ties to even: 1+2^-8 -> 1 (even), 1+2^-7+2^-8 -> 1+2^-6 (even), below half -> down
    want = np.array([1.0, 1.0, 1.0 + 2 ** -6, 1.0, -2.5, np.inf, -np.inf, 2.9999e38],
                    np.float64)
    got = O.bf16_round(x).astype(np.float64)
    assert np.array_equal(got[:7], want[:7])
    assert abs(got[7] - 3.0e38) / 3.0e38 < 2 ** -8
    assert O.bf16_bits(np.array([np.nan], np.float32))[0] == 0x7FC0


def test_bf16_round_is_nearest():
    x = _rng(1).standard_normal(10000).astype(np.float32)
    r = O.bf16_round(x).astype(np.float64)
    # nearest: error at most half a bf16 ulp (8 explicit mantissa bits)
    ulp = 2.0 ** (np.floor(np.log2(np.abs(x))) - 7)
    assert (np.abs(r - x) <= ulp / 2 + 1e-30).all()
    assert np.array_equal(O.bf16_round(r.astype(np.float32)), r.astype(np.float32))


# ---------------------------------------------------------------------- gating

def test_gating_matches_float64_closed_form():
    rng = _rng(2)
    A_log = rng.uniform(-3, 3, O.HV).astype(np.float32)
    dt_bias = rng.uniform(-1, 1, O.HV).astype(np.float32)
    a = (3 * rng.standard_normal((50, O.HV))).astype(np.float32)
    b = (3 * rng.standard_normal((50, O.HV))).astype(np.float32)
    g, beta = O.gating(A_log, a, dt_bias, b)
    for t in range(50):
        for h in range(O.HV):
            x = float(a[t, h]) + float(dt_bias[h])
            sp = x if x > 20 else math.log1p(math.exp(x))
            want_g = math.exp(-math.exp(float(A_log[h])) * sp)
            want_b = 1.0 / (1.0 + math.exp(-float(b[t, h])))
            # float32 exponent of size L carries a relative error of ~L * 2^-24
            tol = 4e-7 * max(1.0, abs(math.log(max(want_g, 1e-300)))) * want_g + 1e-38
            assert abs(g[t, h] - want_g) <= tol
            assert abs(beta[t, h] - want_b) <= 2e-7


def test_gating_limits():
    A_log = np.zeros(O.HV, np.float32)
    dt = np.zeros(O.HV, np.float32)
    # softplus threshold: x > 20 is the identity (F.softplus threshold=20)
    x = np.full((1, O.HV), 25.0, np.float32)
    assert np.allclose(O.log_decay(A_log, x, dt), -25.0, rtol=0, atol=0)
    x = np.full((1, O.HV), 20.0, np.float32)
    assert np.allclose(O.log_decay(A_log, x, dt), -math.log1p(math.exp(20.0)), rtol=1e-7)
    # A_log -> -inf means no decay
    g, _ = O.gating(np.full(O.HV, -np.inf, np.float32), np.ones((1, O.HV), np.float32), dt,
                    np.zeros((1, O.HV), np.float32))
    assert np.all(g == 1.0)
    # beta -> {0, 1} at b -> -/+ inf and 0.5 at 0
    b = np.zeros((1, O.HV), np.float32)
    b[0, :3] = [-np.inf, 0.0, np.inf]
    _, beta = O.gating(A_log, np.zeros((1, O.HV), np.float32), dt, b)
    assert beta[0, :3].tolist() == [0.0, 0.5, 1.0]


def test_resolve_scale():
    assert O.resolve_scale(None) == 1 / math.sqrt(128)
    assert O.resolve_scale(0.0) == 1 / math.sqrt(128)
    assert O.resolve_scale(0.5) == 0.5
    assert O.resolve_scale(np.float32(2.0)) == 2.0


# ---------------------------------------------------------------------- decode

def _decode_inputs_f64(B, seed, normalize=True):
    rng = _rng(seed)
    q = rng.standard_normal((B, 1, O.H_QK, O.DK))
    k = rng.standard_normal((B, 1, O.H_QK, O.DK))
    if normalize:
        q /= np.linalg.norm(q, axis=-1, keepdims=True)
        k /= np.linalg.norm(k, axis=-1, keepdims=True)
    v = rng.standard_normal((B, 1, O.HV, O.DV))
    S = 0.05 * rng.standard_normal((B, O.HV, O.DV, O.DK))
    A_log = rng.uniform(0, math.log(16), O.HV)
    a = rng.standard_normal((B, 1, O.HV))
    dt = rng.uniform(0, 1, O.HV)
    b = rng.standard_normal((B, 1, O.HV))
    return q, k, v, S, A_log, a, dt, b


def test_decode_zero_state_closed_form():
    q, k, v, _, A_log, a, dt, b = _decode_inputs_f64(3, 10)
    scale = 0.3
    o, S = O.decode(q, k, v, None, A_log, a, dt, b, scale, dtype=np.float64)
    beta = 1 / (1 + np.exp(-b[:, 0]))  # [B,HV]
    for n in range(3):
        for h in range(O.HV):
            kh, qh, vh = k[n, 0, h // 2], q[n, 0, h // 2], v[n, 0, h]
            want_S = beta[n, h] * np.outer(vh, kh)  # k-last: S[v, k]
            assert np.allclose(S[n, h], want_S, rtol=0, atol=1e-13)
            want_o = scale * beta[n, h] * (kh @ qh) * vh
            assert np.allclose(o[n, 0, h], O.bf16_round(want_o.astype(np.float32)), atol=0)


def test_decode_beta_zero_is_pure_decay():
    q, k, v, S0, A_log, a, dt, _ = _decode_inputs_f64(2, 11)
    b = np.full((2, 1, O.HV), -np.inf)
    scale = 0.7
    o, S = O.decode(q, k, v, S0, A_log, a, dt, b, scale, dtype=np.float64)
    g = np.exp(-np.exp(A_log) * np.log1p(np.exp(a[:, 0] + dt)))
    for n in range(2):
        for h in range(O.HV):
            want = g[n, h] * S0[n, h]
            assert np.allclose(S[n, h], want, rtol=1e-12, atol=1e-14 * np.abs(want).max())
            want_o = scale * g[n, h] * (S0[n, h] @ q[n, 0, h // 2])  # o[v] = sum_k S[v,k] q[k]
            assert np.allclose(o[n, 0, h], O.bf16_round(want_o.astype(np.float32)), atol=0)


def test_decode_delta_overwrite_identity():
    # |k| = 1 and beta = 1: the new state maps k exactly to v (S'' k = v).
    q, k, v, S0, A_log, a, dt, _ = _decode_inputs_f64(2, 12)
    b = np.full((2, 1, O.HV), np.inf)
    _, S = O.decode(q, k, v, S0, A_log, a, dt, b, 1.0, dtype=np.float64)
    for n in range(2):
        for h in range(O.HV):
            assert np.allclose(S[n, h] @ k[n, 0, h // 2], v[n, 0, h], atol=1e-12)


def test_decode_gva_head_map():
    # v-head h must read q/k head h // 2: replacing every q/k head by head
    # h // 2 leaves v-head h unchanged.
    q, k, v, S0, A_log, a, dt, b = _decode_inputs_f64(2, 13)
    o, S = O.decode(q, k, v, S0, A_log, a, dt, b, 0.5, dtype=np.float64)
    for h in range(O.HV):
        qs = np.repeat(q[:, :, h // 2:h // 2 + 1], O.H_QK, axis=2)
        ks = np.repeat(k[:, :, h // 2:h // 2 + 1], O.H_QK, axis=2)
        o2, S2 = O.decode(qs, ks, v, S0, A_log, a, dt, b, 0.5, dtype=np.float64)
        assert np.array_equal(S[:, h], S2[:, h])
        assert np.array_equal(o[:, :, h], o2[:, :, h])
    # and the heads are really distinct (the check above is not vacuous)
    assert not np.allclose(S[:, 0], S[:, 2])


def test_decode_loop_equals_batched():
    inp = O.make_decode_inputs(3, seed=5)
    o1, s1 = O.decode(**inp)
    o2, s2 = O.decode_loop(**inp)
    assert np.abs(s1 - s2).max() < 1e-6
    assert np.abs(o1 - o2).max() <= 2 ** -7 * np.abs(o1).max()


def test_decode_fp32_tracks_fp64():
    inp = O.make_decode_inputs(4, seed=6)
    o32, s32 = O.decode(**inp)
    o64, s64 = O.decode(**inp, dtype=np.float64)
    assert np.abs(s32 - s64).max() < 1e-6
    assert np.abs(o32 - o64).max() <= 1e-2


# --------------------------------------------------------------------- prefill

def _prefill_from_decode_steps(inp, lens):
    """L decode steps of the decode oracle per sequence (float64)."""
    cu = np.concatenate([[0], np.cumsum(lens)])
    outs, states = [], []
    for s, L in enumerate(lens):
        S = None if inp["state"] is None else inp["state"][s:s + 1].astype(np.float64)
        if L == 0:
            states.append(np.zeros((1, O.HV, O.DV, O.DK)))
            continue
        for t in range(cu[s], cu[s + 1]):
            o, S = O.decode(inp["q"][t][None, None], inp["k"][t][None, None],
                            inp["v"][t][None, None], S, inp["A_log"], inp["a"][t][None, None],
                            inp["dt_bias"], inp["b"][t][None, None], inp["scale"],
                            dtype=np.float64)
            outs.append(o[0, 0])
        states.append(S)
    return np.stack(outs) if outs else np.zeros((0, O.HV, O.DV)), np.concatenate(states)


@pytest.mark.parametrize("lens", [[1], [5], [3, 0, 4]])
def test_prefill_equals_decode_steps(lens):
    inp = O.make_prefill_inputs(lens, seed=20)
    o, S = O.prefill_seq(**inp, dtype=np.float64)
    o2, S2 = _prefill_from_decode_steps(inp, lens)
    assert np.allclose(S, S2, rtol=0, atol=1e-13)
    assert np.array_equal(o, o2)


def test_prefill_split_invariance():
    inp = O.make_prefill_inputs([70], seed=21)
    o, S = O.prefill_seq(**inp, dtype=np.float64)
    first = {k: (v[:30] if k in ("q", "k", "v", "a", "b") else v) for k, v in inp.items()}
    first["cu_seqlens"] = np.array([0, 30])
    o1, S1 = O.prefill_seq(**first, dtype=np.float64)
    second = {k: (v[30:] if k in ("q", "k", "v", "a", "b") else v) for k, v in inp.items()}
    second["cu_seqlens"] = np.array([0, 40])
    second["state"] = S1
    o2, S2 = O.prefill_seq(**second, dtype=np.float64)
    assert np.allclose(S, S2, rtol=0, atol=1e-13)
    assert np.array_equal(o, np.concatenate([o1, o2]))


def test_prefill_packing_invariance_and_zero_length():
    lens = [9, 0, 17, 5]
    inp = O.make_prefill_inputs(lens, seed=22)
    o, S = O.prefill_seq(**inp)
    assert np.all(S[1] == 0.0), "a zero-length sequence must leave a zero state"
    cu = inp["cu_seqlens"]
    for s in range(len(lens)):
        sl = slice(cu[s], cu[s + 1])
        one = {k: (v[sl] if k in ("q", "k", "v", "a", "b") else v) for k, v in inp.items()}
        one["cu_seqlens"] = np.array([0, lens[s]])
        one["state"] = inp["state"][s:s + 1]
        o1, S1 = O.prefill_seq(**one)
        assert np.array_equal(o[sl], o1)
        if lens[s]:
            assert np.array_equal(S[s], S1[0])


@pytest.mark.parametrize("cu", [[0, 100], [20, 90], [7, 7, 50, 110], [64, 64], [33]])
def test_prefill_partial_cu_is_a_shifted_batch(cu):
    # offsets that do not span [0, T) (reference/gdn_prefill_ref.py:49-62):
    # the rows outside [cu[0], cu[N]) stay zero, and the covered rows equal
    # the same batch cut out of the buffer with offsets shifted to start at 0
    # (checked in C and numpy, so both oracles follow the reference here).
    T = 128
    N = len(cu) - 1
    inp = O.make_prefill_inputs([T], seed=24, with_state=False)
    rng = np.random.default_rng(25)
    inp["state"] = (0.05 * rng.standard_normal((N, O.HV, O.DV, O.DK))).astype(np.float32)
    inp["cu_seqlens"] = np.array(cu, np.int64)
    lo, hi = cu[0], cu[-1]
    cut = {k: (v[lo:hi] if k in ("q", "k", "v", "a", "b") else v) for k, v in inp.items()}
    cut["cu_seqlens"] = np.array(cu, np.int64) - lo
    o_cut, S_cut = O.prefill_seq(**cut)
    for fn in (O.prefill_seq, O.prefill_seq_c):
        o, S = fn(**inp)
        assert not o[:lo].any() and not o[hi:].any()
        if hi > lo:
            assert np.abs(o[lo:hi] - o_cut).max() <= 2 ** -7 * np.abs(o_cut).max()
        assert S.shape == S_cut.shape and (N == 0 or np.abs(S - S_cut).max() < 1e-6)


def test_prefill_state_none_equals_zero_state():
    inp = O.make_prefill_inputs([12, 7], seed=23, with_state=False)
    o1, S1 = O.prefill_seq(**inp)
    inp["state"] = np.zeros((2, O.HV, O.DV, O.DK), np.float32)
    o2, S2 = O.prefill_seq(**inp)
    assert np.array_equal(o1, o2) and np.array_equal(S1, S2)


# ----------------------------------------------------------- chunked WY form

@pytest.mark.parametrize("lens", [[1], [63], [64], [65], [127, 128], [200, 0, 31]])
def test_chunked_equals_sequential_f64(lens):
    inp = O.make_prefill_inputs(lens, seed=30)
    o, S = O.prefill_chunked(**inp)
    o_seq, S_seq = O.prefill_seq(**inp, dtype=np.float64)
    assert np.abs(S - S_seq).max() < 1e-10
    # the sequential oracle rounds o to bf16, the chunked one does not
    assert np.abs(O.bf16_round(o.astype(np.float32)) - o_seq).max() <= \
        2 ** -8 * np.abs(o_seq).max()


def test_chunked_equals_sequential_slow_decay():
    inp = O.make_prefill_inputs([300], seed=31, slow_decay_heads=(6, 7))
    _, S = O.prefill_chunked(**inp)
    _, S_seq = O.prefill_seq(**inp, dtype=np.float64)
    assert np.abs(S - S_seq).max() < 1e-10


def test_chunked_intermediates():
    inp = O.make_prefill_inputs([64, 100], seed=32)
    _, _, it = O.prefill_chunked(**inp, return_intermediates=True)
    glog = O.log_decay(inp["A_log"], inp["a"], inp["dt_bias"], np.float64)
    # chunk 2 = second sequence's first chunk (tokens 64..127)
    assert np.allclose(it["g_cs"][1, 3], np.cumsum(glog[64:128, 3]), rtol=1e-14)
    for c in range(3):
        for h in (0, 5):
            C = 64 if c < 2 else 36
            A = it["A"][c, h, :C, :C]
            assert np.all(np.triu(A) == 0.0), "A must be strictly lower triangular"
            Ai = it["Ai"][c, h, :C, :C]
            want = scipy.linalg.solve_triangular(np.eye(C) + A, np.eye(C), lower=True,
                                                 unit_diagonal=True)
            assert np.allclose(Ai, want, rtol=1e-12, atol=1e-12)
            assert np.allclose(Ai @ (np.eye(C) + A), np.eye(C), atol=1e-11)


# ---------------------------------------------------------------- chunk index

def _brute_chunks(lens):
    seq, local = [], []
    for s, L in enumerate(lens):
        c = 0
        for t in range(0, L, O.CHUNK):
            seq.append(s)
            local.append(c)
            c += 1
    return seq, local


@pytest.mark.parametrize("lens", [[1], [64], [65], [0, 64, 0, 1, 130], [6, 49, 294, 1800, 2040, 61],
                                  [0], [0, 0]])
def test_chunk_index_brute_force(lens):
    cu = np.concatenate([[0], np.cumsum(lens)])
    seq, local, offs = O.chunk_index(cu)
    bs, bl = _brute_chunks(lens)
    assert seq.tolist() == bs and local.tolist() == bl
    assert offs[-1] == len(bs)
    assert offs.tolist() == [0] + np.cumsum([-(-L // 64) for L in lens]).tolist()
    assert O.max_chunks(sum(lens), len(lens)) >= len(bs)


def test_chunk_index_rejects_decreasing():
    with pytest.raises(ValueError):
        O.chunk_index([0, 5, 3])


def test_max_chunks_bound_is_tight_and_safe():
    rng = _rng(40)
    for _ in range(300):
        N = int(rng.integers(1, 12))
        lens = rng.integers(0, 300, N)
        T = int(lens.sum())
        nt = int(sum(-(-int(L) // 64) for L in lens))
        assert O.max_chunks(T, N) >= nt
    # tight: N sequences of 1 token need N chunks; one long one needs ceil(T/64)
    assert O.max_chunks(7, 7) == 7
    assert O.max_chunks(8192, 1) == 128


# ---------------------------------------------------------------- C oracle

def test_c_oracle_matches_numpy():
    inp = O.make_prefill_inputs([6, 49, 0, 70], seed=50)
    o1, S1 = O.prefill_seq(**inp)
    o2, S2 = O.prefill_seq_c(**inp)
    assert np.abs(S1 - S2).max() < 1e-6
    assert np.abs(o1 - o2).max() <= 2 ** -7 * np.abs(o1).max()
    o3, S3 = O.prefill_seq(**inp, dtype=np.float64)
    o4, S4 = O.prefill_seq_c(**inp, use_f64=True)
    assert np.abs(S3 - S4).max() < 1e-6  # the C f64 path stores float32
    inp["state"] = None
    o5, S5 = O.prefill_seq(**inp)
    o6, S6 = O.prefill_seq_c(**inp)
    assert np.abs(S5 - S6).max() < 1e-6


def test_input_recipe():
    inp = O.make_decode_inputs(2, seed=0)
    assert np.allclose(np.linalg.norm(inp["q"], axis=-1), 1.0, atol=1e-2)
    assert np.array_equal(O.bf16_round(inp["q"]), inp["q"])
    assert inp["state"].dtype == np.float32
    assert (inp["A_log"] >= 0).all() and (inp["A_log"] <= math.log(16)).all()
    p = O.make_prefill_inputs([3, 4], seed=1, slow_decay_heads=(6, 7))
    assert p["cu_seqlens"].tolist() == [0, 3, 7]
    assert p["A_log"][6] == -10.0 and p["A_log"][7] == -10.0


def test_work_formulas():
    assert O.decode_bytes(64) == 67_504_192
    assert O.decode_bytes(1) == 1_054_816
    assert O.prefill_bytes(8192, 1) == 51_642_448
    assert O.prefill_flops(128) == 128 * 8 * 11_534_336


# ---------------------------------------------------------------------------
# generalised head configurations (q/k heads HQK, v-heads HV = multiple of HQK)
# ---------------------------------------------------------------------------

HEAD_CONFIGS = [(16, 32), (2, 8), (1, 1)]


@pytest.mark.parametrize("heads", HEAD_CONFIGS)
def test_decode_general_heads_equals_per_head_problems(heads):
    # Each v-head h is an independent single-head problem on q/k head
    # h // (HV / HQK): a wrong head map (h % HQK, h // 2, ...) fails here.
    hqk, hv = heads
    inp = O.make_decode_inputs(3, seed=5, heads=heads)
    o, s = O.decode(**inp)
    ratio = hv // hqk
    for h in range(hv):
        one = dict(inp)
        for n in ("q", "k"):
            one[n] = inp[n][:, :, h // ratio:h // ratio + 1]
        one["v"] = inp["v"][:, :, h:h + 1]
        one["a"] = inp["a"][:, :, h:h + 1]
        one["b"] = inp["b"][:, :, h:h + 1]
        one["A_log"] = inp["A_log"][h:h + 1]
        one["dt_bias"] = inp["dt_bias"][h:h + 1]
        one["state"] = inp["state"][:, h:h + 1]
        o1, s1 = O.decode(**one)
        np.testing.assert_array_equal(o[:, :, h:h + 1], o1)
        np.testing.assert_array_equal(s[:, h:h + 1], s1)


@pytest.mark.parametrize("heads", [(16, 32), (2, 8)])
def test_prefill_general_heads_chained_decode_and_c(heads):
    # prefill(L) == L decode steps, the C recurrence == numpy, and the chunked
    # float64 form == the sequential one, at a non-reference head layout.
    lens = [5, 0, 70]
    inp = O.make_prefill_inputs(lens, seed=9, heads=heads)
    o_seq, s_seq = O.prefill_seq(**inp, dtype=np.float64)
    o_c, s_c = O.prefill_seq_c(**inp, use_f64=True)  # gating in float32 there
    assert np.abs(s_c - s_seq).max() <= 1e-6 * np.abs(s_seq).max()
    o_ch, s_ch = O.prefill_chunked(**inp)
    assert np.abs(s_ch - s_seq).max() <= 1e-9 * np.abs(s_seq).max()
    assert np.abs(o_ch - o_seq).max() <= 1e-2 * np.abs(o_seq).max()
    cu = inp["cu_seqlens"]
    for s_i, L in enumerate(lens):
        st = inp["state"][s_i:s_i + 1].astype(np.float64)
        for t in range(cu[s_i], cu[s_i + 1]):
            step = {n: inp[n][t:t + 1][:, None] for n in ("q", "k", "v", "a", "b")}
            o1, st = O.decode(state=st, A_log=inp["A_log"], dt_bias=inp["dt_bias"],
                              scale=inp["scale"], dtype=np.float64, **step)
            np.testing.assert_allclose(o1[0, 0], o_seq[t], rtol=1e-2, atol=1e-2)
        want = st[0] if L > 0 else np.zeros_like(st[0])
        assert np.abs(s_seq[s_i] - want).max() <= 1e-9 * max(np.abs(want).max(), 1.0)
