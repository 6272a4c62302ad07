"""ctypes binding of libgdn_amd.so (the C ABI declared in include/gdn_amd.h).

The library is built in-tree (``make -C gated-delta-network_amd/csrc`` or
``__graft_entry__.build()``).  There is no fallback: if the library is missing
or does not export a symbol, loading raises, so no caller can silently run
anything but the HIP kernels.
"""

from __future__ import annotations

import ctypes
import os

LIB_NAME = "libgdn_amd.so"
LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), LIB_NAME)

GDN_OK = 0
GDN_ERR_INVALID = -1
GDN_ERR_LAUNCH = -2
GDN_ERR_WORKSPACE = -3
PREFILL_SCRATCH_BYTES = 64 << 20  # GDN_PREFILL_SCRATCH_BYTES
ABI_VERSION = 4

_P = ctypes.c_void_p
_I = ctypes.c_int
_F = ctypes.c_float
_SZ = ctypes.c_size_t

# name -> (restype, argtypes); mirrors include/gdn_amd.h one to one.
SIGNATURES = {
    "gdn_abi_version": (_I, []),
    "gdn_last_error": (ctypes.c_char_p, []),
    "gdn_decode_fwd": (_I, [_P, _P, _P, _P, _P, _P, _P, _P, _F, _P, _P, _I, _P]),
    "gdn_decode_fwd_variant": (_I, [_P, _P, _P, _P, _P, _P, _P, _P, _F, _P, _P, _I, _P, _I]),
    "gdn_decode_multi_fwd": (_I, [_P, _P, _P, _P, _P, _P, _P, _P, _F, _P, _P, _I, _I, _P, _I]),
    "gdn_decode_fwd_heads": (_I, [_P, _P, _P, _P, _P, _P, _P, _P, _F, _P, _P, _I, _I, _I, _I,
                                  _P, _I]),
    "gdn_prefill_workspace_bytes": (_SZ, [_I, _I]),
    "gdn_prefill_workspace_bytes_heads": (_SZ, [_I, _I, _I, _I]),
    "gdn_prefill_fwd": (_I, [_P, _P, _P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _F, _P, _P, _P,
                             _SZ, _P]),
    "gdn_prefill_fwd_variant": (_I, [_P, _P, _P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _F, _P, _P,
                                     _P, _SZ, _P, _I]),
    "gdn_prefill_fwd_tuned": (_I, [_P, _P, _P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _F, _P, _P,
                                   _P, _SZ, _P, _I, _I, _I]),
    "gdn_prefill_fwd_heads": (_I, [_P, _P, _P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _F,
                                   _P, _P, _P, _SZ, _P, _I, _I, _I]),
    "gdn_prefill_fwd_noalloc": (_I, [_P, _P, _P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _F, _P, _P,
                                     _P]),
    "gdn_prefill_status_offset": (ctypes.c_longlong, [_I, _I, _I, _I]),
    "gdn_prefill_status": (_I, [_P, _I, _I, _I, _I, _P, _P]),
    "gdn_stream_copy": (_I, [_P, _P, _SZ, _P]),
}


class GdnError(RuntimeError):
    """A launch or runtime failure reported by the HIP library."""


class GdnWorkspaceError(GdnError):
    """The prefill workspace was missing or too small."""


_lib = None


def load(path: str = LIB_PATH) -> ctypes.CDLL:
    """Load (once) and return the HIP library with every prototype set."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(path):
        raise RuntimeError(
            f"{path} is not built; build it with `make -C gated-delta-network_amd/csrc` "
            "or `python -c 'import __graft_entry__ as g; g.build()'`")
    lib = ctypes.CDLL(path)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)  # AttributeError if the symbol is missing
        fn.restype = res
        fn.argtypes = args
    got = lib.gdn_abi_version()
    if got != ABI_VERSION:
        raise RuntimeError(f"{path}: ABI version {got}, expected {ABI_VERSION}")
    _lib = lib
    return lib


def last_error() -> str:
    return load().gdn_last_error().decode(errors="replace")


def check(rc: int, what: str) -> None:
    """Turn a GDN_* status into the matching Python exception."""
    if rc == GDN_OK:
        return
    msg = last_error() or what
    if rc == GDN_ERR_INVALID:
        raise ValueError(msg)
    if rc == GDN_ERR_WORKSPACE:
        raise GdnWorkspaceError(msg)
    raise GdnError(f"{msg} (status {rc})")
