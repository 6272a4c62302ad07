"""Entry point of the HIP solution for gdn_decode_qk4_v8_d128_k_last.

Drop-in for the reference's solutions/gdn_decode_qk4_v8_d128_k_last/solution/*/kernel.py::kernel: same
destination-passing signature; the work runs in hand-written gfx950 kernels.
"""

import os
import sys

_HERE = os.path.dirname(os.path.abspath(__file__))
# Unpacked from solution.json, this file sits at the root of the packed tree
# beside gated-delta-network_amd/; in the repository it is four levels below it.
_PACKED = os.path.join(_HERE, "gated-delta-network_amd")
_PKG = _PACKED if os.path.isdir(_PACKED) else os.path.abspath(
    os.path.join(_HERE, *([os.pardir] * 4)))
if _PKG not in sys.path:
    sys.path.insert(0, _PKG)

if _PKG == _PACKED:  # sources only: build libgdn_amd.so once with hipcc
    from gdn_amd.packing import ensure_library  # noqa: E402

    ensure_library()

from gdn_amd.decode import kernel  # noqa: E402,F401

__all__ = ["kernel"]
