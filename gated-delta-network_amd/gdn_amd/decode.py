"""Decode entry point: the reference's destination-passing ``kernel(...)``.

Same name, argument order and meaning as
solutions/gdn_decode_qk4_v8_d128_k_last/solution/triton/kernel.py:85 and
solution/cuda/binding.py:195, with the semantics of
reference/gdn_decode_ref.py:12-83 (state may be None; scale None/0.0 means
1/sqrt(128)).  The work is one launch of the HIP kernel behind
``gdn_decode_fwd`` (include/gdn_amd.h) on torch's current stream.

Beyond the reference (whose decode asserts T == 1 and 4/8 heads): tensors
with T > 1 tokens per row ([B, T, ...], multi-token / speculative decode) run
the tokens in order through ``gdn_decode_multi_fwd``, the state written once
at the end; other head layouts (q/k heads from ``q``, v-heads from ``v``, the
latter a multiple of the former) run through ``gdn_decode_fwd_heads``.
"""

from __future__ import annotations

import torch

from . import _lib
from ._common import (DK, DV, H_QK, HV, check_output, check_tensor, dense, fast_ok,
                      resolve_scale, stream_of)

_BF = torch.bfloat16
_F32 = torch.float32
_DTYPES = (_BF, _BF, _BF, _F32, _BF, _F32, _BF, _BF, _F32)


def _heads(q, v):
    """(q/k heads, v-heads) of a call: 4 and 8 for the reference definition."""
    hqk = q.shape[2] if isinstance(q, torch.Tensor) and q.dim() == 4 else H_QK
    hv = v.shape[2] if isinstance(v, torch.Tensor) and v.dim() == 4 else HV
    return hqk, hv


def _validate(q, k, v, state, A_log, a, dt_bias, b, output, new_state):
    if not isinstance(q, torch.Tensor) or q.dim() != 4 or q.shape[1] < 1:
        raise ValueError("q must be a [B, T, 4, 128] tensor with T >= 1")
    B, T = q.shape[0], q.shape[1]
    dev = q.device
    if dev.type != "cuda":
        raise ValueError(f"q is on {dev}; the HIP kernels need device tensors")
    H_QK, HV = _heads(q, v)
    if H_QK < 1 or HV < 1 or HV % H_QK:
        raise ValueError(f"v-heads ({HV}) must be a multiple of q/k heads ({H_QK})")
    bf, f32 = torch.bfloat16, torch.float32
    check_tensor("q", q, (B, T, H_QK, DK), bf, dev)
    check_tensor("k", k, (B, T, H_QK, DK), bf, dev)
    check_tensor("v", v, (B, T, HV, DV), bf, dev)
    if state is not None:
        check_tensor("state", state, (B, HV, DV, DK), f32, dev)
    check_tensor("A_log", A_log, (HV,), f32, dev)
    check_tensor("a", a, (B, T, HV), bf, dev)
    check_tensor("dt_bias", dt_bias, (HV,), f32, dev)
    check_tensor("b", b, (B, T, HV), bf, dev)
    check_tensor("output", output, (B, T, HV, DV), bf, dev)
    check_tensor("new_state", new_state, (B, HV, DV, DK), f32, dev)
    check_output("output", output)
    check_output("new_state", new_state)
    return B, dev


def kernel(q, k, v, state, A_log, a, dt_bias, b, scale, output, new_state, *, variant=-1):
    """GDN decode of T tokens per row (T=1: one step), written into ``output``
    and ``new_state``.

    q, k [B,T,4,128] bf16; v [B,T,8,128] bf16; state [B,8,128,128] f32 k-last
    or None; A_log, dt_bias [8] f32; a, b [B,T,8] bf16; scale float, 0-d
    tensor or None; output [B,T,8,128] bf16; new_state [B,8,128,128] f32.
    ``new_state`` may be ``state`` itself (in-place update).  ``variant``
    picks a tiling (gdn_decode_fwd_variant for T=1, gdn_decode_multi_fwd for
    T>1: 0..9 token by token, 10 the 16-token block kernel); the default is
    the built-in one.
    """
    lib = _lib.load()
    four = isinstance(q, torch.Tensor) and q.dim() == 4
    B = q.shape[0] if four else -1
    T = q.shape[1] if four else -1
    H_QK, HV = _heads(q, v)
    ts = (q, k, v, A_log, a, dt_bias, b, output, new_state)
    shapes = ((B, T, H_QK, DK), (B, T, H_QK, DK), (B, T, HV, DV), (HV,), (B, T, HV), (HV,),
              (B, T, HV), (B, T, HV, DV), (B, HV, DV, DK))
    if B < 0 or T < 1 or not (fast_ok(ts, _DTYPES, shapes) and
                     (state is None or fast_ok((q, state), (_BF, _F32),
                                               (shapes[0], shapes[-1])))):
        _validate(q, k, v, state, A_log, a, dt_bias, b, output, new_state)
        if state is not None and state.data_ptr() != new_state.data_ptr():
            state = dense(state)
        q, k, v, a, b, A_log, dt_bias = (dense(t) for t in (q, k, v, a, b, A_log, dt_bias))
    dev = q.device
    scale = resolve_scale(scale)
    args = (q.data_ptr(), k.data_ptr(), v.data_ptr(),
            None if state is None else state.data_ptr(), A_log.data_ptr(), a.data_ptr(),
            dt_bias.data_ptr(), b.data_ptr(), scale, output.data_ptr(), new_state.data_ptr(),
            B)
    if (H_QK, HV) != (4, 8):
        rc = lib.gdn_decode_fwd_heads(*args, T, H_QK, HV, stream_of(dev), int(variant))
        _lib.check(rc, "gdn_decode_fwd_heads")
        return
    if T > 1:
        rc = lib.gdn_decode_multi_fwd(*args, T, stream_of(dev), int(variant))
        _lib.check(rc, "gdn_decode_multi_fwd")
        return
    args = args + (stream_of(dev),)
    if variant == -1:
        rc = lib.gdn_decode_fwd(*args)
    else:
        rc = lib.gdn_decode_fwd_variant(*args, int(variant))
    _lib.check(rc, "gdn_decode_fwd")


def run(q, k, v, state, A_log, a, dt_bias, b, scale):
    """Non-DPS form with the reference's return convention
    (reference/gdn_decode_ref.py:12, returns (output, new_state))."""
    B, T = q.shape[0], q.shape[1]
    HV = v.shape[2]
    output = torch.empty((B, T, HV, DV), dtype=torch.bfloat16, device=q.device)
    new_state = torch.empty((B, HV, DV, DK), dtype=torch.float32, device=q.device)
    kernel(q, k, v, state, A_log, a, dt_bias, b, scale, output, new_state)
    return output, new_state
