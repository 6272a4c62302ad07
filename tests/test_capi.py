"""The C-ABI library: it loads, exports every symbol include/gdn_amd.h
declares, and rejects bad arguments before touching the GPU (no device
needed; nothing here launches a kernel)."""

import ctypes
import os
import re

import pytest

from gdn_amd import _lib

HEADER = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))),
                      "include", "gdn_amd.h")


def _declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(gdn_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_the_entry_points():
    names = _declared_functions()
    for want in ("gdn_decode_fwd", "gdn_prefill_fwd", "gdn_prefill_workspace_bytes",
                 "gdn_last_error", "gdn_abi_version"):
        assert want in names


def test_library_exports_every_declared_symbol():
    lib = ctypes.CDLL(_lib.LIB_PATH)
    for name in _declared_functions():
        assert hasattr(lib, name), f"{name} declared in gdn_amd.h but not exported"
        assert name in _lib.SIGNATURES, f"{name} has no ctypes prototype"


def test_abi_version_and_load():
    lib = _lib.load()
    assert lib.gdn_abi_version() == _lib.ABI_VERSION


def _decode_args(**over):
    args = dict(q=1 << 20, k=2 << 20, v=3 << 20, state=None, A_log=4 << 20, a=5 << 20,
                dt_bias=6 << 20, b=7 << 20, scale=0.1, output=8 << 20, new_state=16 << 20,
                batch=1, stream=None)
    args.update(over)
    return list(args.values())


DECODE_BAD = [
    (dict(q=None), "null"),
    (dict(output=None), "null"),
    (dict(batch=-1), "batch"),
    (dict(scale=0.0), "scale"),
    (dict(scale=float("nan")), "scale"),
    (dict(scale=float("inf")), "scale"),
    (dict(new_state=(16 << 20) + 4), "aligned"),
    (dict(q=(1 << 20) + 2), "aligned"),
    (dict(output=(3 << 20) + 256), "overlap"),
    (dict(state=(16 << 20) + 1024), "overlap"),
]


@pytest.mark.parametrize("over, needle", DECODE_BAD)
def test_decode_rejects_bad_arguments(over, needle):
    lib = _lib.load()
    rc = lib.gdn_decode_fwd(*_decode_args(**over))
    assert rc == _lib.GDN_ERR_INVALID
    assert needle in _lib.last_error()


def test_decode_zero_batch_is_a_no_op():
    lib = _lib.load()
    assert lib.gdn_decode_fwd(*_decode_args(batch=0)) == _lib.GDN_OK


def test_decode_unknown_variant():
    lib = _lib.load()
    rc = lib.gdn_decode_fwd_variant(*_decode_args(), 15)
    assert rc == _lib.GDN_ERR_INVALID and "variant" in _lib.last_error()


def test_check_maps_status_to_exceptions():
    _lib.check(_lib.GDN_OK, "x")
    with pytest.raises(ValueError):
        _lib.check(_lib.GDN_ERR_INVALID, "x")
    with pytest.raises(_lib.GdnWorkspaceError):
        _lib.check(_lib.GDN_ERR_WORKSPACE, "x")
    with pytest.raises(_lib.GdnError):
        _lib.check(_lib.GDN_ERR_LAUNCH, "x")


def _prefill_args(**over):
    args = dict(q=1 << 20, k=2 << 20, v=3 << 20, state=None, A_log=4 << 20, a=5 << 20,
                dt_bias=6 << 20, b=7 << 20, cu=8 << 20, cu64=1, N=2, T=100, scale=0.1,
                output=16 << 20, new_state=32 << 20, ws=64 << 20, ws_bytes=1 << 30, stream=None)
    args.update(over)
    return list(args.values())


def test_prefill_workspace_bytes():
    lib = _lib.load()
    assert lib.gdn_prefill_workspace_bytes(0, 0) >= 0
    assert lib.gdn_prefill_workspace_bytes(-1, 1) == 0
    small = lib.gdn_prefill_workspace_bytes(64, 1)
    big = lib.gdn_prefill_workspace_bytes(8192, 1)
    assert 0 < small < big
    # bounded by the chunk count alone: 1x8192 -> 128 chunks (~120 MiB of
    # per-chunk operands, plus 17.5 MiB for the two-segment scan of one sequence)
    assert big < 144 * 2 ** 20
    assert lib.gdn_prefill_workspace_bytes(8192, 4) > lib.gdn_prefill_workspace_bytes(8192, 2)


PREFILL_BAD = [
    (dict(cu=None), "cu_seqlens", _lib.GDN_ERR_INVALID),
    (dict(q=None), "null", _lib.GDN_ERR_INVALID),
    (dict(N=-1), "num_seqs", _lib.GDN_ERR_INVALID),
    (dict(scale=-1.0), "scale", _lib.GDN_ERR_INVALID),
    (dict(q=(1 << 20) + 8), "aligned", _lib.GDN_ERR_INVALID),
    (dict(ws_bytes=16), "workspace", _lib.GDN_ERR_WORKSPACE),
    (dict(ws=None), "workspace", _lib.GDN_ERR_WORKSPACE),
    (dict(output=(3 << 20) + 64), "overlap", _lib.GDN_ERR_INVALID),
    (dict(ws=(1 << 20)), "overlap", _lib.GDN_ERR_INVALID),
    (dict(output=(16 << 20) + 2), "aligned", _lib.GDN_ERR_INVALID),
    (dict(cu=(8 << 20) + 4), "cu_seqlens", _lib.GDN_ERR_INVALID),
]


@pytest.mark.parametrize("over, needle, code", PREFILL_BAD)
def test_prefill_rejects_bad_arguments(over, needle, code):
    lib = _lib.load()
    rc = lib.gdn_prefill_fwd(*_prefill_args(**over))
    assert rc == code
    assert needle in _lib.last_error()


def test_prefill_no_sequences_is_a_no_op():
    lib = _lib.load()
    assert lib.gdn_prefill_fwd(*_prefill_args(N=0, T=0)) == _lib.GDN_OK


def _multi_args(**over):
    args = dict(q=1 << 20, k=2 << 20, v=3 << 20, state=None, A_log=4 << 20, a=5 << 20,
                dt_bias=6 << 20, b=7 << 20, scale=0.1, output=8 << 20, new_state=16 << 20,
                batch=2, tokens=3, stream=None, variant=-1)
    args.update(over)
    return list(args.values())


MULTI_BAD = [
    (dict(tokens=0), "tokens"),
    (dict(batch=-1), "batch"),
    (dict(v=None), "null"),
    (dict(scale=0.0), "scale"),
    (dict(variant=11), "variant"),
    (dict(variant=-2), "variant"),
    (dict(new_state=(16 << 20) + 8), "aligned"),
    # output is [B*T, 8, 128] bf16 = 12 KiB: ending inside v
    (dict(output=(3 << 20) - 4096), "overlap"),
    (dict(state=(16 << 20) + 4096), "overlap"),
    (dict(v=(3 << 20) + 1), "2-byte"),
    # the block kernel's 16-byte row loads
    (dict(q=(1 << 20) + 8, variant=10), "block kernel"),
    (dict(v=(3 << 20) + 8, variant=10), "block kernel"),
]


@pytest.mark.parametrize("over, needle", MULTI_BAD)
def test_decode_multi_rejects_bad_arguments(over, needle):
    lib = _lib.load()
    rc = lib.gdn_decode_multi_fwd(*_multi_args(**over))
    assert rc == _lib.GDN_ERR_INVALID
    assert needle in _lib.last_error()


def test_decode_multi_zero_batch_is_a_no_op():
    lib = _lib.load()
    assert lib.gdn_decode_multi_fwd(*_multi_args(batch=0)) == _lib.GDN_OK


TUNED_BAD = [
    ((-1, -3, -1), "recurrent_max_len"),
    ((-1, -1, 11), "recurrent tiling"),
    ((5, -1, -1), "variant"),
    ((-2, -1, -1), "variant"),
]


@pytest.mark.parametrize("tuning, needle", TUNED_BAD)
def test_prefill_tuned_rejects_bad_tuning(tuning, needle):
    lib = _lib.load()
    rc = lib.gdn_prefill_fwd_tuned(*_prefill_args(), *tuning)
    assert rc == _lib.GDN_ERR_INVALID
    assert needle in _lib.last_error()


def _heads_args(hqk, hv):
    return _multi_args()[:-2] + [hqk, hv, None, -1]


@pytest.mark.parametrize("hqk, hv", [(3, 8), (0, 8), (4, 0), (2048, 2048), (8, 4)])
def test_decode_heads_rejects_bad_heads(hqk, hv):
    lib = _lib.load()
    rc = lib.gdn_decode_fwd_heads(*_heads_args(hqk, hv))
    assert rc == _lib.GDN_ERR_INVALID
    assert "heads" in _lib.last_error()


def test_decode_heads_zero_batch_is_a_no_op():
    lib = _lib.load()
    args = _multi_args(batch=0)[:-2] + [16, 32, None, -1]
    assert lib.gdn_decode_fwd_heads(*args) == _lib.GDN_OK


def test_prefill_workspace_bytes_heads():
    lib = _lib.load()
    for T, N in ((0, 0), (64, 1), (8192, 1), (8192, 4), (300, 7)):
        assert lib.gdn_prefill_workspace_bytes_heads(T, N, 4, 8) == \
            lib.gdn_prefill_workspace_bytes(T, N)
    assert lib.gdn_prefill_workspace_bytes_heads(8192, 1, 16, 32) > \
        lib.gdn_prefill_workspace_bytes(8192, 1)
    for hqk, hv in ((3, 8), (0, 8), (4, 0), (2048, 2048)):
        assert lib.gdn_prefill_workspace_bytes_heads(64, 1, hqk, hv) == 0


def test_prefill_status_offset():
    # the status words follow the chunk table and the offsets/flags region,
    # each region on a 256-byte boundary (prefill_layout, gdn_args.cpp)
    lib = _lib.load()
    up = lambda n: (n + 255) // 256 * 256
    for T, N in [(1, 1), (1000, 1), (8192, 4), (4250, 6), (100, 300), (0, 5)]:
        nt = min(T, (T + 63 * N) // 64) if T and N else 0
        assert lib.gdn_prefill_status_offset(T, N, 4, 8) == up(nt * 16) + up((N + 3) * 4)
        assert lib.gdn_prefill_status_offset(T, N, 4, 8) + 4 * N <= \
            lib.gdn_prefill_workspace_bytes(T, N)
    for T, N, hqk, hv in [(-1, 1, 4, 8), (10, 0, 4, 8), (10, 1, 3, 8), (10, 1, 0, 8)]:
        assert lib.gdn_prefill_status_offset(T, N, hqk, hv) == -1


def test_prefill_status_rejects_bad_arguments():
    lib = _lib.load()
    got = ctypes.c_int(0)
    assert lib.gdn_prefill_status(None, 10, 1, 4, 8, None, None) == _lib.GDN_ERR_INVALID
    assert "gdn_prefill_status" in _lib.last_error()
    assert lib.gdn_prefill_status(None, 10, 0, 4, 8, None, ctypes.byref(got)) == _lib.GDN_ERR_INVALID


@pytest.mark.parametrize("hqk, hv", [(3, 8), (0, 8), (8, 4)])
def test_prefill_heads_rejects_bad_heads(hqk, hv):
    lib = _lib.load()
    a = _prefill_args()
    rc = lib.gdn_prefill_fwd_heads(*a[:12], hqk, hv, *a[12:], -1, -1, -1)
    assert rc == _lib.GDN_ERR_INVALID
    assert "heads" in _lib.last_error()


@pytest.mark.parametrize("src, dst, nbytes, needle", [
    (None, 1 << 20, 32768, "null"),
    (1 << 20, (1 << 21) + 8, 32768, "aligned"),
    (1 << 20, 1 << 21, 32768 + 16, "multiple"),
    (1 << 20, (1 << 20) + 16384, 32768, "overlap"),
])
def test_stream_copy_rejects_bad_arguments(src, dst, nbytes, needle):
    # Rejected before any HIP call, so this runs without a GPU.
    lib = _lib.load()
    assert lib.gdn_stream_copy(src, dst, nbytes, None) == _lib.GDN_ERR_INVALID
    assert needle in _lib.last_error()
