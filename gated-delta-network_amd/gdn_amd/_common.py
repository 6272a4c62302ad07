"""Argument handling shared by the decode and prefill entry points."""

from __future__ import annotations

import math

import torch

H_QK = 4
HV = 8
DK = 128
DV = 128
CHUNK = 64


def resolve_scale(scale, head_size: int = DK) -> float:
    """Scale as the reference resolves it.

    A tensor scale is read with ``.item()`` (solutions/gdn_decode_qk4_v8_d128_k_last/
    solution/triton/kernel.py:92-93); ``None`` or ``0.0`` means 1/sqrt(head_size)
    (reference/gdn_decode_ref.py:38-39, gdn_prefill_ref.py:38-39).
    """
    if isinstance(scale, torch.Tensor):
        scale = scale.item()
    if scale is None or scale == 0.0:
        return 1.0 / math.sqrt(head_size)
    scale = float(scale)
    if not math.isfinite(scale) or scale <= 0.0:
        raise ValueError(f"scale must be a finite positive number, got {scale}")
    return scale


def check_tensor(name: str, t, shape, dtype, device) -> None:
    if not isinstance(t, torch.Tensor):
        raise ValueError(f"{name} must be a torch.Tensor, got {type(t).__name__}")
    if t.dtype != dtype:
        raise ValueError(f"{name} must be {dtype}, got {t.dtype}")
    if tuple(t.shape) != tuple(shape):
        raise ValueError(f"{name} must have shape {tuple(shape)}, got {tuple(t.shape)}")
    if t.device != device:
        raise ValueError(f"{name} is on {t.device}, expected {device}")


def dense(t: torch.Tensor) -> torch.Tensor:
    """Inputs may be strided views; the kernels read dense row-major copies
    (the reference's own wrappers call .contiguous(), triton/kernel.py:99-103)."""
    return t if t.is_contiguous() else t.contiguous()


def check_output(name: str, t: torch.Tensor) -> None:
    if not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous: it is written in place")


_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def stream_of(device: torch.device) -> int:
    """Handle of torch's current stream on `device` (a hipStream_t on ROCm)."""
    if _raw_stream is not None:
        return _raw_stream(device.index if device.index is not None else 0)
    return torch.cuda.current_stream(device).cuda_stream


def fast_ok(tensors, dtypes, shapes) -> bool:
    """Cheap all-in-one check run before the detailed, message-producing one:
    every tensor on one CUDA device, with the given dtype and shape, and
    dense.  False means "run the detailed validation"."""
    Tensor = torch.Tensor
    dev = tensors[0].get_device() if isinstance(tensors[0], Tensor) else -1
    if dev < 0:
        return False
    for t, dt, sh in zip(tensors, dtypes, shapes):
        if (not isinstance(t, Tensor) or t.dtype is not dt or t.shape != sh
                or t.get_device() != dev or not t.is_contiguous()):
            return False
    return True
