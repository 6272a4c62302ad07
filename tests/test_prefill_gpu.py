"""Prefill parity on the GPU: the HIP pipeline (through the C ABI, via the DPS
entry point) against the CPU oracle on the same seeded inputs.

Tolerance (stated once in conftest.py): bf16 output atol = rtol = 1e-2; f32
final state atol = 1e-3 * max|state_ref|.  The oracle is the sequential
recurrence (oracle/gdn_seq.c, pinned against the numpy restatement and the
float64 chunked form in tests/test_oracle.py).  Stage checks compare the
workspace intermediates with the float64 chunked oracle.
"""

import importlib.util
import math
import os

import numpy as np
import pytest
import torch

from conftest import PKG, assert_output_close, assert_state_close
from oracle import gdn_oracle as O

pytestmark = pytest.mark.gpu

SOLUTION = os.path.join(PKG, "solutions", "gdn_prefill_qk4_v8_d128_k_last", "solution", "hip",
                        "kernel.py")


def _entry():
    spec = importlib.util.spec_from_file_location("gdn_prefill_solution", SOLUTION)
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod.kernel


kernel = _entry()


def to_dev(inp, dev, cu_dtype=torch.int64):
    bf = torch.bfloat16
    d = {n: torch.from_numpy(np.ascontiguousarray(inp[n])).to(dev).to(bf)
         for n in ("q", "k", "v", "a", "b")}
    for n in ("A_log", "dt_bias"):
        d[n] = torch.from_numpy(inp[n]).to(dev)
    d["state"] = None if inp["state"] is None else torch.from_numpy(inp["state"]).to(dev)
    d["cu_seqlens"] = torch.from_numpy(inp["cu_seqlens"]).to(dev).to(cu_dtype)
    d["scale"] = inp["scale"]
    return d


# "auto": the built-in per-sequence routing (short sequences token by token);
# "chunked": every sequence through the chunk-64 pipeline.
ROUTES = {"auto": -1, "chunked": -2}


def run_gpu(d, dev, in_place=False, variant=None, route="auto"):
    T = d["q"].shape[0]
    N = d["cu_seqlens"].numel() - 1
    out = torch.empty((T, 8, 128), dtype=torch.bfloat16, device=dev)
    ns = d["state"] if in_place else torch.empty((N, 8, 128, 128), dtype=torch.float32, device=dev)
    args = (d["q"], d["k"], d["v"], d["state"], d["A_log"], d["a"], d["dt_bias"], d["b"],
            d["cu_seqlens"], d["scale"], out, ns)
    if variant is None and route == "auto":
        kernel(*args)
    else:
        from gdn_amd import prefill
        prefill.kernel(*args, variant=-1 if variant is None else variant,
                       recurrent_max_len=ROUTES[route])
    torch.cuda.synchronize()
    return out.float().cpu().numpy(), ns.cpu().numpy()


def check(o, s, o_ref, s_ref):
    assert_output_close(o, o_ref)
    assert_state_close(s, s_ref)


# The reference's own prefill cases (tests/test_prefill.py:196-217) and the
# configurations of its benchmark script (scripts/benchmark.py:131-142).
REFERENCE_CASES = [
    ([32], False), ([64], False), ([128], False), ([256], False), ([31], False), ([65], False),
    ([127], False), ([64, 64], False), ([32, 96], False), ([64, 128], False),
    ([64], True), ([128], True), ([64, 128], True),
    ([512], True), ([1024], True), ([128, 128], True), ([256, 256], True),
    ([32, 64, 128, 256], True),
]


@pytest.mark.parametrize("route", list(ROUTES))
@pytest.mark.parametrize("lens, with_state", REFERENCE_CASES)
def test_prefill_reference_cases(cuda_device, lens, with_state, route):
    print(f"prefill parity lens={lens} state={with_state} route={route}", flush=True)
    inp = O.make_prefill_inputs(lens, seed=100 + len(lens), with_state=with_state)
    o_ref, s_ref = O.prefill_seq_c(**inp)
    o, s = run_gpu(to_dev(inp, cuda_device), cuda_device, route=route)
    check(o, s, o_ref, s_ref)


@pytest.mark.parametrize("route", list(ROUTES))
@pytest.mark.parametrize("lens", [[1], [2, 1, 3], [63], [0, 5, 0, 70], [0], [0, 0, 17],
                                  [129, 0, 1, 64, 65]])
def test_prefill_edge_lengths(cuda_device, lens, route):
    print(f"prefill edge lens={lens} route={route}", flush=True)
    inp = O.make_prefill_inputs(lens, seed=7)
    o_ref, s_ref = O.prefill_seq_c(**inp)
    o, s = run_gpu(to_dev(inp, cuda_device), cuda_device, route=route)
    for i, L in enumerate(lens):
        if L == 0:
            assert np.all(s[i] == 0.0), "zero-length sequence must give a zero state"
    check(o, s, o_ref, s_ref)


@pytest.mark.parametrize("route", list(ROUTES))
def test_prefill_many_sequences_multi_tile_index(cuda_device, route):
    # > 1024 sequences: the chunk-index scan runs over several tiles.
    rng = np.random.default_rng(11)
    lens = rng.integers(0, 4, 1500).tolist()
    lens[0] = 70
    lens[700] = 300
    inp = O.make_prefill_inputs(lens, seed=8)
    o_ref, s_ref = O.prefill_seq_c(**inp)
    o, s = run_gpu(to_dev(inp, cuda_device), cuda_device, route=route)
    check(o, s, o_ref, s_ref)


def test_prefill_config2_1x1024(cuda_device):
    cfg = O.CONFIGS["prefill_1x1024"]
    inp = O.make_prefill_inputs(cfg["lens"], seed=cfg["seed"], with_state=cfg["with_state"])
    o_ref, s_ref = O.prefill_seq_c(**inp)
    o, s = run_gpu(to_dev(inp, cuda_device), cuda_device)
    check(o, s, o_ref, s_ref)


def test_prefill_config3_varlen(cuda_device):
    cfg = O.CONFIGS["prefill_varlen6"]
    inp = O.make_prefill_inputs(cfg["lens"], seed=cfg["seed"], with_state=cfg["with_state"])
    o_ref, s_ref = O.prefill_seq_c(**inp)
    o, s = run_gpu(to_dev(inp, cuda_device), cuda_device)
    check(o, s, o_ref, s_ref)


def test_prefill_1x8192(cuda_device):
    cfg = O.CONFIGS["prefill_1x8192"]
    inp = O.make_prefill_inputs(cfg["lens"], seed=cfg["seed"], with_state=cfg["with_state"])
    o_ref, s_ref = O.prefill_seq_c(**inp)
    o, s = run_gpu(to_dev(inp, cuda_device), cuda_device)
    check(o, s, o_ref, s_ref)


def test_prefill_config4_long_context(cuda_device):
    cfg = O.CONFIGS["prefill_4x8192"]
    inp = O.make_prefill_inputs(cfg["lens"], seed=cfg["seed"], with_state=cfg["with_state"],
                                slow_decay_heads=cfg["slow_decay_heads"])
    o_ref, s_ref = O.prefill_seq_c(**inp)
    o, s = run_gpu(to_dev(inp, cuda_device), cuda_device)
    check(o, s, o_ref, s_ref)


# Forms of the per-chunk operands (variant): 0 WY, 1 T.
FORMS = {"wy": 0, "t": 1}
CHAIN_WY, SPLIT_WY = 2, 3  # WY with one serial chain / with the two-segment scan


def form_rule(lens, hv=8):
    """Restatement of the built-in form choice of gdn_prefill.hip (index
    kernel, t_form_wins in gdn_common.h): the T form from 144 chunks on for a
    batch holding more than three times the chunks of its longest sequence,
    or from 384 on with at least 1.5 times; and for batches of at most 768
    state units (sequence, v-head, 16 columns) whose longest sequence has at
    most 12 chunks, with more than one sequence holding chunks."""
    chunks = [-(-L // 64) for L in lens]
    nt, longest, units = sum(chunks), max(chunks), len(lens) * hv * 8
    large = nt >= 144 and (nt > 3 * longest or (nt >= 384 and nt >= 1.5 * longest))
    small = units <= 768 and longest <= 12 and nt > longest
    return 1 if large or small else 0


@pytest.mark.parametrize("form", list(FORMS))
def test_prefill_forms_reference_and_edge_cases(cuda_device, form):
    # Every reference case and edge length through the chunks in both forms.
    cases = [(lens, st) for lens, st in REFERENCE_CASES] + \
        [(lens, True) for lens in ([1], [2, 1, 3], [63], [0, 5, 0, 70], [0], [0, 0, 17],
                                   [129, 0, 1, 64, 65], [100, 0, 300])]
    for i, (lens, with_state) in enumerate(cases):
        print(f"prefill form={form} lens={lens} state={with_state}", flush=True)
        inp = O.make_prefill_inputs(lens, seed=300 + i, with_state=with_state)
        o_ref, s_ref = O.prefill_seq_c(**inp)
        o, s = run_gpu(to_dev(inp, cuda_device), cuda_device, variant=FORMS[form], route="chunked")
        for j, L in enumerate(lens):
            if L == 0:
                assert np.all(s[j] == 0.0), "zero-length sequence must give a zero state"
        check(o, s, o_ref, s_ref)


@pytest.mark.parametrize("lens", [[512] * 16, [1024] * 8, [2048] * 4, [4096] * 2, [8192, 1024, 512, 100],
                                  [6, 49, 294, 1800, 2040, 61], [64] * 130, [512] * 32, [2048] * 8,
                                  [4096, 4096, 4096], [64] * 200, [8192, 64, 4096],
                                  [256] * 4, [384] * 8, [150] * 12, [100, 700], [800, 64, 64],
                                  [128] * 16, [768] * 12])
def test_prefill_built_in_form_choice(cuda_device, lens):
    # The built-in choice is bit-identical to the form the rule names, and
    # the flag the index kernel leaves in the workspace is that form.
    from gdn_amd import prefill
    print(f"prefill form choice lens={len(lens)}x{lens[0]}.. expect {form_rule(lens)}", flush=True)
    inp = O.make_prefill_inputs(lens, seed=21)
    d = to_dev(inp, cuda_device)
    o_a, s_a = run_gpu(d, cuda_device, variant=-1, route="chunked")
    T, N = sum(lens), len(lens)
    L = _layout(T, N)
    ws = prefill._workspace(cuda_device, _stream(cuda_device), 0).cpu().numpy()
    flag = np.frombuffer(ws[L["offsets"]:L["offsets"] + (N + 3) * 4].tobytes(), np.int32)[N + 2]
    assert flag == form_rule(lens)
    o_f, s_f = run_gpu(d, cuda_device, variant=form_rule(lens), route="chunked")
    assert np.array_equal(o_a, o_f) and np.array_equal(s_a, s_f)
    o_ref, s_ref = O.prefill_seq_c(**inp)
    check(o_a, s_a, o_ref, s_ref)


def test_prefill_wy_product_form_ragged_batch(cuda_device):
    # 40 + 47 + 11 + 1 = 99 chunks (partial last chunks in every sequence) x 8
    # v-heads = 792 units: past the 768 from which the WY intra kernel forms w
    # and u as T and two products; the built-in choice keeps the WY form
    # (99 < 144 chunks) and indexes the batch in the intra kernel
    lens = [2500, 3000, 700, 33]
    inp = O.make_prefill_inputs(lens, seed=29)
    print(f"prefill product form lens={lens}", flush=True)
    o, s = run_gpu(to_dev(inp, cuda_device), cuda_device, route="chunked")
    o_ref, s_ref = O.prefill_seq_c(**inp)
    check(o, s, o_ref, s_ref)
    assert form_rule(lens) == 0


@pytest.mark.parametrize("form", list(FORMS))
def test_prefill_self_index_matches_index_kernel(cuda_device, form):
    # A batch of at most 256 sequences and two rounds of intra workgroups
    # builds its chunk table inside the intra kernel; padded with empty
    # sequences to 257 it goes through the index kernel.  Same chunks, same
    # form, same kernels otherwise: bit-identical outputs and states.
    lens = [300, 0, 1000, 64, 5]
    inp = O.make_prefill_inputs(lens, seed=27)
    T, N = sum(lens), len(lens)
    print(f"prefill self index vs index kernel form={form} T={T}", flush=True)
    d = to_dev(inp, cuda_device)
    o_s, s_s = run_gpu(d, cuda_device, variant=FORMS[form], route="chunked")
    pad = 257 - N
    d2 = dict(d)
    d2["cu_seqlens"] = torch.cat([d["cu_seqlens"], torch.full((pad,), T, dtype=d["cu_seqlens"].dtype,
                                                               device=cuda_device)])
    d2["state"] = torch.cat([d["state"], torch.zeros((pad, 8, 128, 128), dtype=torch.float32,
                                                     device=cuda_device)])
    o_i, s_i = run_gpu(d2, cuda_device, variant=FORMS[form], route="chunked")
    assert np.array_equal(o_s, o_i)
    assert np.array_equal(s_s, s_i[:N]) and not s_i[N:].any()
    o_ref, s_ref = O.prefill_seq_c(**inp)
    check(o_s, s_s, o_ref, s_ref)


@pytest.mark.parametrize("form", list(FORMS))
def test_prefill_forms_extreme_gates(cuda_device, form):
    # Per-head gates around softplus' threshold (x > 20), beta saturated at 0
    # and 1, decays ~1 and so fast that exp(G) underflows inside a chunk.
    lens = [200, 64, 130]
    inp = O.make_prefill_inputs(lens, seed=31)
    rng = np.random.default_rng(31)
    T = sum(lens)
    a_h = np.array([30.0, -30.0, 20.0, 0.0, 19.5, -5.0, 5.0, 1.0], np.float32)
    b_h = np.array([-40.0, 40.0, 0.0, 8.0, -8.0, 1.0, -1.0, 0.0], np.float32)
    inp["a"][:] = O.bf16_round(a_h[None, :] + rng.normal(0, 0.5, (T, 8)).astype(np.float32))
    inp["b"][:] = O.bf16_round(b_h[None, :] + rng.normal(0, 0.5, (T, 8)).astype(np.float32))
    inp["A_log"][:] = np.array([-10.0, 2.7, 0.0, -20.0, 1.0, 0.5, 0.1, 2.0], np.float32)
    print(f"prefill extreme gates form={form}", flush=True)
    o_ref, s_ref = O.prefill_seq_c(**inp)
    o, s = run_gpu(to_dev(inp, cuda_device), cuda_device, variant=FORMS[form], route="chunked")
    assert np.isfinite(o).all() and np.isfinite(s).all()
    check(o, s, o_ref, s_ref)


@pytest.mark.parametrize("variant", [0, 1, CHAIN_WY, SPLIT_WY])
def test_prefill_operand_magnitudes(cuda_device, variant):
    # Keys and values far from unit size, per head: the WY form stores w's
    # low half in fp8 under a power-of-two scale taken from max|w| of each
    # (chunk, head), and w scales with k.  q/k head 0 keys x 1e-3, head 1
    # x 0.05; v-heads 0-1 values x 1e4, 2-3 x 1e-4.  Each head's output and
    # state are checked against its own magnitude.
    lens = [700, 130] if variant in (0, 1) else [900]
    inp = O.make_prefill_inputs(lens, seed=33, slow_decay_heads=(7,))
    inp["k"] = O.bf16_round(inp["k"] * np.array([1e-3, 0.05, 1.0, 1.0], np.float32)[None, :, None])
    vs = np.array([1e4, 1e4, 1e-4, 1e-4, 1.0, 1.0, 1.0, 1.0], np.float32)
    inp["v"] = O.bf16_round(inp["v"] * vs[None, :, None])
    if inp["state"] is not None:
        inp["state"] = (inp["state"] * vs[None, :, None, None]).astype(np.float32)
    print(f"prefill operand magnitudes variant={variant} lens={lens}", flush=True)
    o_ref, s_ref = O.prefill_seq_c(**inp)
    o, s = run_gpu(to_dev(inp, cuda_device), cuda_device, variant=variant, route="chunked")
    for h in range(8):
        m = max(float(np.abs(o_ref[:, h]).max()), 1e-30)
        assert_output_close(o[:, h] / m, o_ref[:, h] / m, what=f"output head {h}")
        assert_state_close(s[:, h], s_ref[:, h], what=f"state head {h}")


def test_prefill_forms_long_sequence(cuda_device):
    # One 32768-token sequence (512 chunks, initial state, two near-unit-decay
    # heads) through both forms against one oracle run.
    inp = O.make_prefill_inputs([32768], seed=32, slow_decay_heads=(6, 7))
    o_ref, s_ref = O.prefill_seq_c(**inp)
    d = to_dev(inp, cuda_device)
    for form, var in FORMS.items():
        print(f"prefill 1x32768 form={form}", flush=True)
        o, s = run_gpu(d, cuda_device, variant=var, route="chunked")
        check(o, s, o_ref, s_ref)


@pytest.mark.parametrize("name", ["prefill_1x8192", "prefill_varlen6", "prefill_4x8192"])
def test_prefill_forms_full_size(cuda_device, name):
    # The benchmark configurations at full size in the form the built-in
    # choice does not take for them.
    cfg = O.CONFIGS[name]
    kw = {"slow_decay_heads": cfg["slow_decay_heads"]} if "slow_decay_heads" in cfg else {}
    inp = O.make_prefill_inputs(cfg["lens"], seed=cfg["seed"], with_state=cfg["with_state"], **kw)
    other = 1 - form_rule(cfg["lens"])
    print(f"prefill {name} form={other}", flush=True)
    o_ref, s_ref = O.prefill_seq_c(**inp)
    o, s = run_gpu(to_dev(inp, cuda_device), cuda_device, variant=other, route="chunked")
    check(o, s, o_ref, s_ref)


@pytest.mark.parametrize("route", list(ROUTES))
def test_prefill_int32_cu_seqlens_state_none_in_place(cuda_device, route):
    inp = O.make_prefill_inputs([40, 90, 300], seed=13)
    d64 = to_dev(inp, cuda_device)
    d32 = to_dev(inp, cuda_device, cu_dtype=torch.int32)
    o64, s64 = run_gpu(d64, cuda_device, route=route)
    o32, s32 = run_gpu(d32, cuda_device, route=route)
    assert np.array_equal(o64, o32) and np.array_equal(s64, s32)
    oi, si = run_gpu(d64, cuda_device, in_place=True, route=route)
    assert np.array_equal(o64, oi) and np.array_equal(s64, si)
    inp["state"] = None
    dn = to_dev(inp, cuda_device)
    o_ref, s_ref = O.prefill_seq_c(**inp)
    on, sn = run_gpu(dn, cuda_device, route=route)
    check(on, sn, o_ref, s_ref)


def test_prefill_scale_forms(cuda_device):
    inp = O.make_prefill_inputs([70], seed=14)
    d = to_dev(inp, cuda_device)
    o1, _ = run_gpu(dict(d, scale=None), cuda_device)
    o2, _ = run_gpu(dict(d, scale=0.0), cuda_device)
    o3, _ = run_gpu(dict(d, scale=torch.tensor(1 / math.sqrt(128))), cuda_device)
    assert np.array_equal(o1, o2) and np.array_equal(o1, o3)
    o_ref, s_ref = O.prefill_seq_c(**dict(inp, scale=0.25))
    o4, s4 = run_gpu(dict(d, scale=0.25), cuda_device)
    check(o4, s4, o_ref, s_ref)


def test_prefill_reference_test_distribution(cuda_device):
    # The reference's own recipe (tests/test_prefill.py:106-113): q, k, v ~
    # 0.1 N(0,1) (not normalised), b ~ 0.1 N(0,1), initial state 0.01 N(0,1),
    # scale 1.0.
    rng = np.random.default_rng(42)
    lens = [64, 128]
    T, N = sum(lens), len(lens)
    f = lambda *s: rng.standard_normal(s).astype(np.float32)
    inp = dict(q=O.bf16_round(0.1 * f(T, 4, 128)), k=O.bf16_round(0.1 * f(T, 4, 128)),
               v=O.bf16_round(0.1 * f(T, 8, 128)), state=0.01 * f(N, 8, 128, 128),
               A_log=0.1 * f(8), a=O.bf16_round(0.1 * f(T, 8)), dt_bias=0.1 * f(8),
               b=O.bf16_round(0.1 * f(T, 8)), cu_seqlens=np.array([0, 64, 192]), scale=1.0)
    o_ref, s_ref = O.prefill_seq_c(**inp)
    o, s = run_gpu(to_dev(inp, cuda_device), cuda_device)
    check(o, s, o_ref, s_ref)


@pytest.mark.parametrize("route", list(ROUTES))
def test_prefill_deterministic(cuda_device, route):
    inp = O.make_prefill_inputs([200, 77, 400], seed=15)
    d = to_dev(inp, cuda_device)
    runs = [run_gpu(d, cuda_device, route=route) for _ in range(3)]
    for o, s in runs[1:]:
        assert np.array_equal(o, runs[0][0]) and np.array_equal(s, runs[0][1])


def test_prefill_then_decode_continues_the_sequence(cuda_device):
    # prefill(L) then one decode step == prefill(L + 1)  (the state is the
    # resumable checkpoint between the two operators)
    from gdn_amd import decode
    L = 100
    inp = O.make_prefill_inputs([L + 1], seed=16)
    o_ref, s_ref = O.prefill_seq_c(**inp)
    first = {n: (x[:L] if n in ("q", "k", "v", "a", "b") else x) for n, x in inp.items()}
    first["cu_seqlens"] = np.array([0, L])
    d = to_dev(first, cuda_device)
    o_pre, s_pre = run_gpu(d, cuda_device)
    dev = cuda_device
    st = torch.from_numpy(s_pre).to(dev)
    step = lambda n: torch.from_numpy(np.ascontiguousarray(inp[n][L:L + 1])).to(dev).to(torch.bfloat16)
    out = torch.empty((1, 1, 8, 128), dtype=torch.bfloat16, device=dev)
    decode.kernel(step("q")[None], step("k")[None], step("v")[None], st,
                  torch.from_numpy(inp["A_log"]).to(dev), step("a")[None],
                  torch.from_numpy(inp["dt_bias"]).to(dev), step("b")[None], inp["scale"], out, st)
    torch.cuda.synchronize()
    o = np.concatenate([o_pre, out.float().cpu().numpy()[0]])
    check(o, st.cpu().numpy(), o_ref, s_ref)


def test_prefill_rejects_bad_arguments(cuda_device):
    inp = O.make_prefill_inputs([10], seed=17)
    d = to_dev(inp, cuda_device)
    out = torch.empty((10, 8, 128), dtype=torch.bfloat16, device=cuda_device)
    ns = torch.empty((1, 8, 128, 128), dtype=torch.float32, device=cuda_device)
    with pytest.raises(ValueError, match="cu_seqlens"):
        kernel(d["q"], d["k"], d["v"], d["state"], d["A_log"], d["a"], d["dt_bias"], d["b"],
               d["cu_seqlens"].float(), d["scale"], out, ns)
    with pytest.raises(ValueError, match="shape"):
        kernel(d["q"][:5], d["k"], d["v"], d["state"], d["A_log"], d["a"], d["dt_bias"], d["b"],
               d["cu_seqlens"], d["scale"], out, ns)


# ------------------------------------------------------------------ stages

def _layout(T, N):
    """Mirror of the workspace layout of gdn_prefill.hip (prefill_layout)."""
    nt = O.max_chunks(T, N)
    off = 0
    L = {"nt": nt}

    def take(name, nbytes):
        nonlocal off
        L[name] = off
        off = (off + nbytes + 255) // 256 * 256

    take("chunks", nt * 16)
    take("offsets", (N + 3) * 4)  # offsets[0..N], then the path and form flags
    take("status", N * 4)         # the cu_seqlens contract bits of each sequence
    take("G", nt * 8 * 64 * 4)
    take("dcy", nt * 8 * 64 * 4)
    take("eg", nt * 8 * 4)
    take("w", nt * 8 * 64 * 128 * 4)  # WY: w; T form: (I + A)^-1
    take("u", nt * 8 * 64 * 128 * 4)  # WY: u; T form: beta, beta exp(G)
    take("kt", nt * 4 * 128 * 64 * 2)
    take("ht", nt * 8 * 128 * 128 * 2)
    take("vnt", nt * 8 * 128 * 64 * 2)
    n1 = nt - (nt + 1) // 2 if N == 1 else 0   # chunks of the second segment
    one = 1 if N == 1 else 0
    take("htm", n1 * 8 * 128 * 128 * 2)
    take("send", one * 8 * 128 * 128 * 4)
    take("cend", one * 8 * 128 * 128 * 4)
    take("mend", one * 8 * 128 * 128 * 4)
    # early output of the two-segment scan: a progress word per first-segment
    # unit (8 v-heads x 8 column blocks), then a done flag per (chunk, v-head)
    # of the first segment
    take("early", one * ((nt + 1) // 2 + 8) * 8 * 4)
    L["total"] = off
    return L


# Stage batches: a small ragged one (32 (chunk, v-head) units: the WY intra
# kernel's two forward substitutions), and one of 121 chunks = 968 units,
# past the 768 (kIntraGemmMinUnits, gdn_prefill.hip) from which the WY intra
# kernel forms T = (I + A)^-1 and w, u as two products instead.
STAGE_BATCHES = {
    "small": [100, 0, 64, 5],
    "product_form": [630, 0, 641] + [640] * 10,
}


@pytest.mark.parametrize("batch", list(STAGE_BATCHES))
@pytest.mark.parametrize("form", list(FORMS))
def test_prefill_stage_intermediates(cuda_device, form, batch):
    from gdn_amd import _lib, prefill
    lens = STAGE_BATCHES[batch]
    print(f"stage intermediates form={form} batch={batch}", flush=True)
    inp = O.make_prefill_inputs(lens, seed=18)
    T, N = sum(lens), len(lens)
    L = _layout(T, N)
    assert prefill.workspace_bytes(T, N) == L["total"]
    d = to_dev(inp, cuda_device)
    run_gpu(d, cuda_device, variant=FORMS[form], route="chunked")
    ws = prefill._workspace(cuda_device, _stream(cuda_device), 0).cpu().numpy()
    _, _, it = O.prefill_chunked(**inp, return_intermediates=True)
    seq, local, offs = O.chunk_index(inp["cu_seqlens"])
    nt = int(offs[-1])
    assert (nt * 8 >= 768) == (batch == "product_form")

    def arr(name, dtype, shape):
        n = int(np.prod(shape))
        return np.frombuffer(ws[L[name]:L[name] + n * np.dtype(dtype).itemsize].tobytes(),
                             dtype=dtype).reshape(shape)

    chunks = arr("chunks", np.int32, (L["nt"], 4))
    assert chunks[:nt, 0].tolist() == seq.tolist()
    assert chunks[:nt, 3].tolist() == local.tolist()
    assert (chunks[nt:, 0] == -1).all()
    flags = arr("offsets", np.int32, (N + 3,))
    assert flags[:N + 1].tolist() == offs.tolist()
    assert flags[N + 1] == 0 and flags[N + 2] == FORMS[form]  # chunk path, this form
    G = arr("G", np.float32, (L["nt"], 8, 64))[:nt]
    dcy = arr("dcy", np.float32, (L["nt"], 8, 64))[:nt]
    eg = arr("eg", np.float32, (L["nt"], 8))[:nt]
    for c in range(nt):
        C = min(64, lens[seq[c]] - 64 * local[c])
        Gc = it["g_cs"][c, :, :C]
        assert np.allclose(G[c, :, :C], Gc, rtol=1e-5, atol=1e-5)
        # the decay factors from the kernel's own f32 cumsum: with |G| up to
        # ~1e3 in a chunk (strong decay), an f32 cumsum is off a float64 one
        # by ~1e-4 in absolute terms, too much for a 1e-4 relative check of
        # exp(G_last - G) against the float64 oracle
        Gk = G[c, :, :C].astype(np.float64)
        assert np.allclose(dcy[c, :, :C], np.exp(Gk[:, -1:] - Gk), rtol=1e-4, atol=1e-6)
        assert np.allclose(eg[c], np.exp(Gk[:, -1]), rtol=1e-4, atol=1e-7)
    if form == "wy":
        # u: MFMA result tiles [c][h][row tile i][col tile n][lane][r] holding
        # u[16i + 4(lane >> 4) + r][16n + (lane & 15)]
        ut = arr("u", np.float32, (L["nt"], 8, 4, 8, 4, 16, 4))[:nt]  # lane = (g, r16)
        u = ut.transpose(0, 1, 2, 4, 6, 3, 5).reshape(nt, 8, 64, 128)
        assert np.abs(u - it["u"]).max() <= 1e-4 * np.abs(it["u"]).max()
        # w (32 KB per chunk and head): A fragments holding
        # w[16mb + (lane & 15)][32kk + 8(lane >> 4) + e] as hi = bf16 [mb][kk][lane][8]
        # (16 KB), lo = OCP fp8 e4m3 [mb][kk / 2][lane][kk % 2][8] (8 KB), and lo's
        # inverse power-of-two scale (f32 at byte 24576): w = hi + lo * scale
        reg = arr("w", np.uint8, (L["nt"], 8, 32768))[:nt]
        hi = np.ascontiguousarray(reg[..., :16384]).view(np.uint16).reshape(nt, 8, 4, 4, 4, 16, 8)
        lo = _e4m3(reg[..., 16384:24576].reshape(nt, 8, 4, 2, 4, 16, 2, 8))
        lo = lo.transpose(0, 1, 2, 3, 6, 4, 5, 7).reshape(nt, 8, 4, 4, 4, 16, 8)
        inv = np.ascontiguousarray(reg[..., 24576:24580]).view(np.float32)[..., 0]  # [c, h]
        assert (inv > 0).all() and (np.log2(inv) == np.round(np.log2(inv))).all()
        assert np.abs(lo).max() < 128  # the scale keeps e4m3 away from its range end
        wv = (O.bf16_from_bits(hi).astype(np.float64)
              + lo * inv[:, :, None, None, None, None, None])           # [c,h,mb,kk,g,r16,e]
        w = wv.transpose(0, 1, 2, 5, 3, 4, 6).reshape(nt, 8, 64, 128)
        # hi is w rounded to bf16 (nearest), lo its remainder to 4 significant bits
        assert np.abs(w - it["w"]).max() <= 1e-4 * np.abs(it["w"]).max()
        hw = O.bf16_from_bits(hi).transpose(0, 1, 2, 5, 3, 4, 6).reshape(nt, 8, 64, 128)
        assert (hw == O.bf16_round(it["w"].astype(np.float32))).mean() > 0.99
    else:
        # T = (I + A)^-1 in the w region: A fragments [c][h][rt][kk][lane][hi 8 | lo 8]
        # holding T[16rt + (lane & 15)][32kk + 8(lane >> 4) + e]
        # (w region stride per (chunk, head): 64 x 128 x 2 bf16; T fills the first half)
        tf = arr("w", np.uint16, (L["nt"], 8, 64 * 128 * 2))[:nt, :, :64 * 64 * 2]
        tf = tf.reshape(nt, 8, 4, 2, 4, 16, 2, 8)                       # lane = (g, r16)
        tv = (O.bf16_from_bits(tf[..., 0, :]).astype(np.float64)
              + O.bf16_from_bits(tf[..., 1, :]))                       # [c,h,rt,kk,g,r16,e]
        Tm = tv.transpose(0, 1, 2, 5, 3, 4, 6).reshape(nt, 8, 64, 64)
        # (beta, beta e^G) in the u region: [c][h][2][64] (u region stride 64 x 128 f32)
        bb = arr("u", np.float32, (L["nt"], 8, 64 * 128))[:nt, :, :128].reshape(nt, 8, 2, 64)
        beta = 1.0 / (1.0 + np.exp(-inp["b"].astype(np.float64)))
        for c in range(nt):
            C = min(64, lens[seq[c]] - 64 * local[c])
            t0 = int(inp["cu_seqlens"][seq[c]]) + 64 * local[c]
            Gc = it["g_cs"][c, :, :C]
            assert np.allclose(bb[c, :, 0, :C], beta[t0:t0 + C].T, rtol=1e-6, atol=1e-7)
            assert np.allclose(bb[c, :, 1, :C], beta[t0:t0 + C].T * np.exp(Gc), rtol=1e-4, atol=1e-6)
            assert (bb[c, :, :, C:] == 0).all()
            # (I + A)^-1 on the chunk's rows, identity on the padding rows
            Ai = it["Ai"][c, :, :C, :C]
            assert np.abs(Tm[c, :, :C, :C] - Ai).max() <= 1e-4 * max(1.0, np.abs(Ai).max())
            pad = np.zeros((8, 64, 64))
            pad[:, C:, C:] = np.eye(64 - C)
            assert (Tm[c][:, C:, :] == pad[:, C:, :]).all() and (Tm[c][:, :C, C:] == 0).all()
    ht = O.bf16_from_bits(arr("ht", np.uint16, (L["nt"], 8, 128, 128))[:nt])
    assert np.abs(ht - it["h"].transpose(0, 1, 3, 2)).max() <= 1e-2 * np.abs(it["h"]).max()
    vnt = O.bf16_from_bits(arr("vnt", np.uint16, (L["nt"], 8, 128, 64))[:nt])
    assert np.abs(vnt - it["v_new"].transpose(0, 1, 3, 2)).max() <= \
        1e-2 * np.abs(it["v_new"]).max()


def _e4m3(bits):
    """OCP fp8 e4m3 (bias 7, no infinities; 0x7f/0xff are NaN) to float64."""
    bits = np.asarray(bits, np.int64)
    sign = np.where(bits & 0x80, -1.0, 1.0)
    e, m = (bits >> 3) & 0xF, bits & 7
    val = np.where(e == 0, m * 2.0 ** -9, (1.0 + m / 8.0) * 2.0 ** (e - 7.0))
    val = np.where((e == 15) & (m == 7), np.nan, val)
    return sign * val


def _stream(dev):
    from gdn_amd._common import stream_of
    return stream_of(dev)


# Two-segment scan of one sequence (gdn_prefill.hip, SplitScan): the second
# half of the chunks runs beside the first from a zero state and from the
# identity, and the second segment's output and new_state then apply the
# first half's final state.
# variant 3 forces it (one sequence of >= 2 chunks), 2 forbids it; the built-in
# choice takes it from 9 chunks on.
SPLIT, CHAIN = 3, 2


@pytest.mark.parametrize("L, with_state, slow", [
    (65, True, ()), (128, False, ()), (129, True, (6, 7)), (1000, True, (6, 7)),
    (4095, False, (0, 7)), (8192, True, (6, 7))])
def test_prefill_two_segment_scan(cuda_device, L, with_state, slow):
    print(f"prefill two-segment scan L={L} state={with_state} slow={slow}", flush=True)
    inp = O.make_prefill_inputs([L], seed=400 + L % 97, with_state=with_state,
                                slow_decay_heads=slow)
    o_ref, s_ref = O.prefill_seq_c(**inp)
    d = to_dev(inp, cuda_device)
    res = {}
    for var in (SPLIT, CHAIN):
        res[var] = run_gpu(d, cuda_device, variant=var, route="chunked")
        check(*res[var], o_ref, s_ref)
    if with_state:  # in place last: it overwrites d["state"]
        oi, si = run_gpu(d, cuda_device, in_place=True, variant=SPLIT, route="chunked")
        assert np.array_equal(oi, res[SPLIT][0]) and np.array_equal(si, res[SPLIT][1])


@pytest.mark.parametrize("L, expect", [(512, CHAIN), (577, SPLIT), (1024, SPLIT), (8192, SPLIT)])
def test_prefill_two_segment_built_in_choice(cuda_device, L, expect):
    print(f"prefill two-segment choice L={L} expect variant {expect}", flush=True)
    inp = O.make_prefill_inputs([L], seed=41, with_state=True)
    d = to_dev(inp, cuda_device)
    o_a, s_a = run_gpu(d, cuda_device, variant=-1, route="chunked")
    o_e, s_e = run_gpu(d, cuda_device, variant=expect, route="chunked")
    assert np.array_equal(o_a, o_e) and np.array_equal(s_a, s_e)


def test_prefill_two_segment_extreme_gates(cuda_device):
    # The gates of test_prefill_forms_extreme_gates on one 1000-token sequence.
    T = 1000
    inp = O.make_prefill_inputs([T], seed=42)
    rng = np.random.default_rng(42)
    a_h = np.array([30.0, -30.0, 20.0, 0.0, 19.5, -5.0, 5.0, 1.0], np.float32)
    b_h = np.array([-40.0, 40.0, 0.0, 8.0, -8.0, 1.0, -1.0, 0.0], np.float32)
    inp["a"][:] = O.bf16_round(a_h[None, :] + rng.normal(0, 0.5, (T, 8)).astype(np.float32))
    inp["b"][:] = O.bf16_round(b_h[None, :] + rng.normal(0, 0.5, (T, 8)).astype(np.float32))
    inp["A_log"][:] = np.array([-10.0, 2.7, 0.0, -20.0, 1.0, 0.5, 0.1, 2.0], np.float32)
    print("prefill two-segment scan, extreme gates", flush=True)
    o_ref, s_ref = O.prefill_seq_c(**inp)
    o, s = run_gpu(to_dev(inp, cuda_device), cuda_device, variant=SPLIT, route="chunked")
    assert np.isfinite(o).all() and np.isfinite(s).all()
    check(o, s, o_ref, s_ref)


@pytest.mark.parametrize("heads", [(1, 1), (2, 8), (8, 8)])
def test_prefill_two_segment_heads(cuda_device, heads):
    from gdn_amd import prefill
    hqk, hv = heads
    L = 1500
    print(f"prefill two-segment scan heads={heads} L={L}", flush=True)
    inp = O.make_prefill_inputs([L], seed=43, heads=heads)
    o_ref, s_ref = O.prefill_seq_c(**inp)
    d = to_dev(inp, cuda_device)
    for var in (SPLIT, CHAIN):
        out = torch.empty((L, hv, 128), dtype=torch.bfloat16, device=cuda_device)
        ns = torch.empty((1, hv, 128, 128), dtype=torch.float32, device=cuda_device)
        prefill.kernel(d["q"], d["k"], d["v"], d["state"], d["A_log"], d["a"], d["dt_bias"],
                       d["b"], d["cu_seqlens"], d["scale"], out, ns, variant=var,
                       recurrent_max_len=-2)
        torch.cuda.synchronize()
        check(out.float().cpu().numpy(), ns.cpu().numpy(), o_ref, s_ref)


EARLY_TAIL = 15  # kEarlyTail (gdn_common.h); built in from 2 * EARLY_TAIL first-segment chunks


@pytest.mark.parametrize("T, cu, variant", [
    (8192, [0, 8192], SPLIT), (8192, [0, 3000], SPLIT), (4000, [130, 3980], SPLIT),
    (8192, [0, 8192], 4), (8192, [0, 3000], 4)])
def test_prefill_early_output_words(cuda_device, T, cu, variant):
    # Two-segment scan with early output (8 v-heads): while the first
    # segment's chain runs, workgroups added to the state launch compute its
    # output for the chunks below n1 - 15 (n1: the segment's chunks of this
    # sequence) as the chain publishes them, and mark them done; the output
    # launch computes the rest.  After the call every first-segment unit's
    # progress word holds n1 - 2 (published at the segment's last step) below
    # its XCD tag (XCD + 1 in the top byte, one XCD per head: MI355X deals
    # workgroups round-robin over its 8 XCDs), and the done flags are set
    # exactly below n1 - 15: no early workgroup stopped.  The output matches
    # the oracle.  Variant 4 stops each early workgroup after its first chunk
    # (chunk e // 8 of workgroup e): only chunks 0..7 are done early, and the
    # output launch computes the rest of the segment through its fallback.
    from gdn_amd import prefill
    print(f"prefill early output words T={T} cu={cu} variant={variant}", flush=True)
    inp = O.make_prefill_inputs([T], seed=45, with_state=True)
    inp["cu_seqlens"] = np.asarray(cu, dtype=np.int64)
    o_ref, s_ref = O.prefill_seq_c(**inp)
    lay = _layout(T, 1)
    o, s = run_gpu(to_dev(inp, cuda_device), cuda_device, variant=variant, route="chunked")
    check(o, s, o_ref, s_ref)
    ws = prefill._workspace(cuda_device, _stream(cuda_device), 0).cpu().numpy()
    nt0 = (lay["nt"] + 1) // 2
    n1 = min(-(-(cu[1] - cu[0]) // 64), nt0)
    words = np.frombuffer(ws[lay["early"]:lay["early"] + (nt0 + 8) * 8 * 4].tobytes(), np.int32)
    prog, done = words[:64].reshape(8, 8), words[64:].reshape(nt0, 8)
    assert ((prog & 0xffffff) == n1 - 2).all(), prog
    tag = prog >> 24
    assert ((tag >= 1) & (tag <= 8)).all() and (tag == tag[:, :1]).all(), tag
    assert len(np.unique(tag[:, 0])) == 8, tag
    expect = (np.arange(nt0) < n1 - EARLY_TAIL)[:, None]
    if variant == 4:
        expect &= (np.arange(nt0) < 8)[:, None]
    assert np.array_equal(done, np.broadcast_to(expect, done.shape).astype(np.int32)), done[:, 0]


@pytest.mark.parametrize("T, cu", [(8192, [0, 8192]), (6000, [37, 5980])])
def test_prefill_early_output_same_bits(cuda_device, T, cu):
    # A chunk of the first segment gets the same output whether the state
    # launch's early workgroups compute it (variant 3) or the output launch
    # does after they stopped (variant 4: one chunk per workgroup early): the
    # same function on the same operands.
    print(f"prefill early output, same bits either way: T={T} cu={cu}", flush=True)
    inp = O.make_prefill_inputs([T], seed=46, with_state=True)
    inp["cu_seqlens"] = np.asarray(cu, dtype=np.int64)
    d = to_dev(inp, cuda_device)
    o3, s3 = run_gpu(d, cuda_device, variant=SPLIT, route="chunked")
    o4, s4 = run_gpu(d, cuda_device, variant=4, route="chunked")
    assert np.array_equal(o3, o4) and np.array_equal(s3, s4)


def test_prefill_two_segment_stage_intermediates(cuda_device):
    # The workspace after a two-segment call: the first segment's chunk-start
    # states (ht) and v_new (vnt) are those of one chain; send is the state
    # at chunk nt0; for the second segment, ht holds the offsets C_c and htm
    # the linear parts M_c of the maps from chunk nt0, so that
    # S_c = send M_c + C_c is the chain's chunk-start state.
    from gdn_amd import prefill
    L = 300  # 5 chunks: nt0 = 3, the last one partial
    inp = O.make_prefill_inputs([L], seed=44)
    lay = _layout(L, 1)
    assert prefill.workspace_bytes(L, 1) == lay["total"]
    run_gpu(to_dev(inp, cuda_device), cuda_device, variant=SPLIT, route="chunked")
    ws = prefill._workspace(cuda_device, _stream(cuda_device), 0).cpu().numpy()
    _, _, it = O.prefill_chunked(**inp, return_intermediates=True)
    nt, nt0 = 5, 3

    def arr(name, dtype, shape):
        n = int(np.prod(shape))
        return np.frombuffer(ws[lay[name]:lay[name] + n * np.dtype(dtype).itemsize].tobytes(),
                             dtype=dtype).reshape(shape)

    h_ref = it["h"].transpose(0, 1, 3, 2)          # [c, h, v, k]
    vn_ref = it["v_new"].transpose(0, 1, 3, 2)     # [c, h, v, token]
    ht = O.bf16_from_bits(arr("ht", np.uint16, (nt, 8, 128, 128))).astype(np.float64)
    vnt = O.bf16_from_bits(arr("vnt", np.uint16, (nt, 8, 128, 64)))
    assert np.abs(ht[:nt0] - h_ref[:nt0]).max() <= 1e-2 * np.abs(h_ref).max()
    assert np.abs(vnt[:nt0] - vn_ref[:nt0]).max() <= 1e-2 * np.abs(vn_ref).max()
    send = arr("send", np.float32, (8, 128, 128)).astype(np.float64)
    assert np.abs(send - h_ref[nt0]).max() <= 1e-4 * np.abs(h_ref[nt0]).max()
    htm = O.bf16_from_bits(arr("htm", np.uint16, (nt - nt0, 8, 128, 128))).astype(np.float64)
    assert np.array_equal(htm[0], np.broadcast_to(np.eye(128), (8, 128, 128)))  # M at nt0 = I
    assert not ht[nt0].any()                                                   # C at nt0 = 0
    for c in range(nt0, nt):
        S_c = send @ htm[c - nt0] + ht[c]
        assert np.abs(S_c - h_ref[c]).max() <= 1e-2 * np.abs(h_ref[c]).max(), f"chunk {c}"
