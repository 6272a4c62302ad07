"""Entry point of the HIP solution for gdn_decode_qk4_v8_d128_k_last.

Drop-in for the reference's solutions/gdn_decode_qk4_v8_d128_k_last/solution/*/kernel.py::kernel: same
destination-passing signature; the work runs in hand-written gfx950 kernels.
"""

import os
import sys

_PKG = os.path.abspath(os.path.join(os.path.dirname(__file__), *([os.pardir] * 4)))
if _PKG not in sys.path:
    sys.path.insert(0, _PKG)

from gdn_amd.decode import kernel  # noqa: E402,F401

__all__ = ["kernel"]
