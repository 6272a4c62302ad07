"""MI355X (gfx950) Gated DeltaNet operators behind the reference's entry points.

* :func:`gdn_amd.decode.kernel`  -- gdn_decode_qk4_v8_d128_k_last (DPS)
* :func:`gdn_amd.prefill.kernel` -- gdn_prefill_qk4_v8_d128_k_last (DPS)

Both call hand-written HIP kernels in libgdn_amd.so through the C ABI of
include/gdn_amd.h; there is no other code path.
"""

from . import _lib  # noqa: F401

__all__ = ["decode", "prefill"]
