"""The library's host-side code under AddressSanitizer and UndefinedBehaviorSanitizer.

gated-delta-network_amd/csrc/gdn_args.cpp holds every host-side computation
of the C-ABI entry points: argument validation, overlap checks, the prefill
workspace layout (max_chunks, prefill_layout), the prefill path plan and the
multi-token kernel choice.  The library compiles it with the host compiler;
here g++ compiles the same file with -fsanitize=address,undefined
-fno-sanitize-recover=all into tests/sanitize/gdn_host_check.cpp's driver, so
any out-of-bounds access, signed overflow, misaligned access or other UB in
that code aborts the driver.  The driver is fed

  * every bad-argument case of tests/test_capi.py, and its status and message
    must equal the real library's for the same call;
  * the workspace layout for extreme (T, N, heads), equal to the library's
    gdn_prefill_workspace_bytes_heads;
  * a sweep of prefill plans over sizes up to INT_MAX, with spot checks of the
    decisions the kernels rely on.

CPU only: no GPU, no HIP runtime, no pointer is dereferenced.
"""

import itertools
import os
import shutil
import subprocess

import pytest

from gdn_amd import _lib
from test_capi import (DECODE_BAD, MULTI_BAD, PREFILL_BAD, TUNED_BAD, _decode_args, _multi_args,
                       _prefill_args)

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(ROOT, "gated-delta-network_amd", "csrc")
DRIVER = os.path.join(ROOT, "tests", "sanitize", "gdn_host_check.cpp")
INT_MAX = 2 ** 31 - 1


@pytest.fixture(scope="module")
def driver(tmp_path_factory):
    gxx = shutil.which("g++")
    if gxx is None:
        pytest.skip("g++ not found")
    exe = str(tmp_path_factory.mktemp("sanitize") / "gdn_host_check")
    cmd = [gxx, "-std=c++17", "-O1", "-g", "-fno-omit-frame-pointer",
           "-fsanitize=address,undefined", "-fno-sanitize-recover=all",
           "-D__host__=", "-D__device__=", "-I", os.path.join(ROOT, "include"), "-I", CSRC,
           DRIVER, os.path.join(CSRC, "gdn_args.cpp"), "-o", exe]
    r = subprocess.run(cmd, capture_output=True, text=True)
    assert r.returncode == 0, r.stderr

    def run(lines):
        env = dict(os.environ)
        # the sanitizer runtime need not be first in the preload list
        env["ASAN_OPTIONS"] = "verify_asan_link_order=0:detect_leaks=1:abort_on_error=0"
        env["UBSAN_OPTIONS"] = "print_stacktrace=1:halt_on_error=1"
        r = subprocess.run([exe], input="".join(l + "\n" for l in lines), capture_output=True,
                           text=True, env=env, timeout=300)
        assert r.returncode == 0, f"sanitizer run failed ({r.returncode}):\n{r.stderr[-4000:]}"
        out = r.stdout.splitlines()
        assert len(out) == len(lines), r.stdout[-2000:]
        return out

    return run


def _num(x):
    if x is None:
        return "0"
    if isinstance(x, float):
        return repr(x)
    return str(int(x))


def _line(cmd, what, args):
    return " ".join([cmd, what] + [_num(a) for a in args])


def test_checks_match_the_library(driver):
    lib = _lib.load()
    lines, lib_results = [], []

    def add(cmd, what, drv_args, call):
        lines.append(_line(cmd, what, drv_args))
        rc = call()
        lib_results.append((rc, _lib.last_error()))

    for over, _ in DECODE_BAD:
        a = _decode_args(**over)  # ..., new_state, batch, stream
        add("decode", "gdn_decode_fwd", a[:12] + [1, 4, 8], lambda a=a: lib.gdn_decode_fwd(*a))
    for over, _ in MULTI_BAD:
        a = _multi_args(**over)  # ..., batch, tokens, stream, variant
        add("multi", "gdn_decode_multi_fwd", a[:13] + [4, 8, a[14]],
            lambda a=a: lib.gdn_decode_multi_fwd(*a))
    for over, _, _ in PREFILL_BAD:
        a = _prefill_args(**over)  # ..., ws, ws_bytes, stream
        add("prefill", "gdn_prefill_fwd", a[:17] + [-1, -1, -1, 4, 8],
            lambda a=a: lib.gdn_prefill_fwd(*a))
    for tuning, _ in TUNED_BAD:
        a = _prefill_args()
        add("prefill", "gdn_prefill_fwd_tuned", a[:17] + list(tuning) + [4, 8],
            lambda a=a, t=tuning: lib.gdn_prefill_fwd_tuned(*a, *t))
    for hqk, hv in [(3, 8), (0, 8), (8, 4), (2048, 2048)]:
        a = _prefill_args()
        add("prefill", "gdn_prefill_fwd_heads", a[:17] + [-1, -1, -1, hqk, hv],
            lambda a=a, h=(hqk, hv): lib.gdn_prefill_fwd_heads(*a[:12], *h, *a[12:], -1, -1, -1))
    out = driver(lines)
    for line, got, (rc, msg) in zip(lines, out, lib_results):
        drv_rc, drv_msg = got.split("\t")[:2]
        assert rc != _lib.GDN_OK, f"library accepted a bad case: {line}"
        assert (int(drv_rc), drv_msg) == (rc, msg), line


def test_valid_arguments_pass_every_check(driver):
    # calls the library would launch (so only the sanitized driver runs them);
    # every buffer at its own 1 TiB-spaced address
    far = {n: (i + 1) << 40 for i, n in enumerate(
        ("q", "k", "v", "A_log", "a", "dt_bias", "b", "cu", "output", "new_state", "ws"))}
    lines = []
    for T, N in [(0, 0), (5, 0), (1, 1), (96, 1), (8192, 1), (4250, 6), (32768, 4), (1024, 64),
                 (300, 7)]:
        for variant, rec_max, rec_var in [(-1, -1, -1), (0, -2, -1), (1, -2, -1), (3, -2, -1),
                                          (-1, 1 << 20, 10), (-1, 64, 0)]:
            a = _prefill_args(N=N, T=T, ws_bytes=1 << 36, **far)
            lines.append(_line("prefill", "gdn_prefill_fwd", a[:17] + [variant, rec_max, rec_var,
                                                                       4, 8]))
    far.pop("cu"), far.pop("ws")
    for batch, tokens, variant in [(0, 1, -1), (64, 1, -1), (64, 4, -1), (64, 16, -1), (3, 33, 10),
                                   (7, 2, 0)]:
        a = _multi_args(batch=batch, tokens=tokens, variant=variant, **far)
        lines.append(_line("multi", "gdn_decode_multi_fwd", a[:13] + [4, 8, a[14]]))
    out = driver(lines)
    for got, line in zip(out, lines):
        assert got.split("\t")[0] == "0", (line, got)
    # the multi-token kernel choice: decode step (-2) for one token, the token
    # kernel's built-in tiling (-1) for short rows (64 x 4: 17.2 vs 18.9 us by
    # the cost models), blocks (10) for long rows, and an explicit tiling as
    # given
    kernels = [int(got.split("\t")[2]) for got in out[-6:]]
    assert kernels == [-2, -2, -1, 10, 10, 0]
    got = driver([_line("multi", "m", _multi_args(batch=6, tokens=5, **far)[:13] + [4, 8, -1])])
    assert int(got[0].split("\t")[2]) == -1


def test_layout_matches_the_library(driver):
    lib = _lib.load()
    cases = []
    for T, N in itertools.product([0, 1, 63, 64, 65, 1000, 8192, 32768, 1 << 20, INT_MAX],
                                  [0, 1, 2, 7, 64, 1024, INT_MAX]):
        for hqk, hv in [(4, 8), (16, 32), (1, 1), (8, 8), (1, 1024), (3, 8), (4, 0)]:
            cases.append((T, N, hqk, hv))
    out = driver([f"layout {T} {N} {hqk} {hv}" for T, N, hqk, hv in cases])
    for (T, N, hqk, hv), got in zip(cases, out):
        rc, nt_max, total = (int(x) for x in got.split())
        want = lib.gdn_prefill_workspace_bytes_heads(T, N, hqk, hv)
        assert total == want, (T, N, hqk, hv)
        if rc == 0:
            assert nt_max == (0 if T == 0 or N == 0 else min(T, (T + 63 * N) // 64))


def test_plan_sweep(driver):
    sizes = [1, 2, 16, 63, 64, 65, 96, 97, 1000, 2047, 2048, 8192, 32768, 1 << 20, INT_MAX]
    counts = [1, 2, 3, 6, 64, 1000, 1 << 16, INT_MAX]
    tunings = [(-1, -1, -1), (0, -1, -1), (1, -1, -1), (2, -1, -1), (3, -1, -1), (4, -1, -1),
               (-1, -2, -1),
               (-1, 100, -1), (-1, 0, 10), (-1, -1, 10), (-1, -1, 3)]
    cases = [(T, N, 4, 8) + t for T in sizes for N in counts if N <= T for t in tunings]
    cases += [(T, N, 16, 32, -1, -1, -1) for T in sizes for N in counts if N <= T]
    out = driver(["plan " + " ".join(map(str, c)) for c in cases])
    plans = {}
    for c, got in zip(cases, out):
        f = [int(x) for x in got.split()]
        plans[c] = dict(rc=f[0], sequential=f[1], seq_variant=f[2], choose=f[3], single=f[4],
                        form=f[5], nt0=f[6], intra=f[7], state=f[8], split=f[9], out=f[10],
                        intra_split=f[11], loop=f[12], self_index=f[13], early=f[14])
    base = (-1, -1, -1)
    p = plans[(96, 1, 4, 8) + base]
    assert p["sequential"] == 1
    p = plans[(8192, 1, 4, 8) + base]
    assert (p["single"], p["form"], p["nt0"], p["state"], p["split"]) == (1, 0, 64, 192, 512)
    # the first segment's early output: 64 workgroups more in the state
    # launch; the output launch covers the first segment with 15 per head
    assert p["early"] == 64
    assert p["out"] == 15 * 8 + 32 * 8  # first segment's rest + new_state tiles
    assert p["intra_split"] == 0  # 1024 chunk-head pairs fill the CUs
    p = plans[(1000, 1, 4, 8) + base]
    assert p["intra_split"] == 1  # 128 pairs: two halves each
    assert p["nt0"] == 8 and p["early"] == 0  # too few first-segment chunks for early output
    assert p["out"] == 8 * 4 // 8 * 8 * 2 + 32 * 8  # chunk-head pairs + new_state tiles
    assert plans[(8192, 1, 16, 32, -1, -1, -1)]["early"] == 0  # no two-segment scan at 32 v-heads
    assert plans[(8192, 1, 4, 8, 4, -1, -1)] == plans[(8192, 1, 4, 8, 3, -1, -1)]  # 4: as 3
    assert plans[(1000, 1, 4, 8, 4, -1, -1)]["nt0"] == 8  # forced, as 3
    p = plans[(8192, 1, 4, 8, 2, -1, -1)]
    assert p["nt0"] == 0 and p["state"] == 64
    p = plans[(32768, 2, 4, 8) + base]
    assert (p["single"], p["form"], p["choose"]) == (0, -1, 0)  # two 16384s: the T form
    p = plans[(8192, 2, 4, 8) + base]
    assert (p["single"], p["form"], p["choose"]) == (0, 0, 0)  # at most 129 chunks: WY
    p = plans[(32768, 64, 4, 8) + base]
    assert p["form"] == -1  # T form possible: left to the index kernel
    assert plans[(INT_MAX, 1, 4, 8) + base]["rc"] == _lib.GDN_OK  # 2^25 chunks still launch
    assert plans[(INT_MAX, INT_MAX, 4, 8) + base]["rc"] == _lib.GDN_ERR_INVALID  # grid too large
    for c, p in plans.items():
        if p["rc"] == 0 and not p["sequential"]:
            # multiples of 8 so that a unit keeps its XCD; when the device
            # makes the path choice, the state grid is capped at the
            # resident workgroups (2 per CU of 256)
            assert p["state"] % 8 == 0 and p["intra"] % 8 == 0 and p["out"] % 8 == 0, c
            assert p["loop"] == (p["choose"] != 0), c
            # early output only with the two-segment scan of 8 v-heads, from
            # 30 first-segment chunks on, its grid within the 256 CUs
            assert p["early"] in (0, 64), c
            if p["early"]:
                assert c[3] == 8 and p["nt0"] >= 30 and p["state"] + p["early"] <= 256, c
            if p["loop"]:
                assert p["state"] <= 512, c
            # batches of 2..256 sequences and at most 2560 intra workgroups
            # index themselves in the intra kernel
            assert p["self_index"] == (1 < c[1] <= 256 and 0 < p["intra"] <= 2560), c
