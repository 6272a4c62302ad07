"""Prefill entry point: the reference's destination-passing ``kernel(...)``.

Same name, argument order and meaning as
solutions/gdn_prefill_qk4_v8_d128_k_last/solution/triton/fla_kernels.py:1049,
with the semantics of reference/gdn_prefill_ref.py:12-91 (state may be None;
scale None/0.0 means 1/sqrt(128); a zero-length sequence yields a zero
state).  The work is the HIP pipeline behind ``gdn_prefill_fwd``
(include/gdn_amd.h) on torch's current stream.  cu_seqlens is never copied to
the host: the chunk table is built on the device, and the workspace is sized
from (T, N) alone.

Workspace: device memory from torch's caching allocator, kept per (device,
stream) and grown on demand, replacing the reference's module-level buffer
cache (fla_kernels.py:950-957), which was keyed by name only.  A caller that
must not allocate inside the call (HIP graph capture, a serving loop) passes
its own buffer as ``workspace=`` (see ``alloc_workspace``); nothing in the
call then allocates, copies to the host or synchronises, so one captured graph
serves any batch of the same (T, N), including new cu_seqlens contents.  A
graph captured without ``workspace=`` writes into the cached buffer of its
stream; once a capture has used a cached buffer, that buffer is never freed
(a larger call later gets a new one), so the graph can always replay into it.
``release_workspaces()`` hands the other cached buffers back to torch.

Rows of ``output`` outside every sequence (before cu_seqlens[0] or from
cu_seqlens[N] on) are written as zeros, as the reference's zero-filled output.
"""

from __future__ import annotations

import ctypes
import threading

import torch

from . import _lib
from ._common import DK, DV, H_QK, HV, check_output, check_tensor, dense, resolve_scale, stream_of

_ws_lock = threading.Lock()
_workspaces: dict = {}  # (device, stream) -> [buffer, used by a graph capture]
_retired: list = []     # replaced buffers that a captured graph may still write


def workspace_bytes(total_tokens: int, num_seqs: int, heads=(H_QK, HV)) -> int:
    """Workspace bytes for T tokens in N sequences with (q/k heads, v-heads)."""
    lib = _lib.load()
    if tuple(heads) == (H_QK, HV):
        return int(lib.gdn_prefill_workspace_bytes(int(total_tokens), int(num_seqs)))
    return int(lib.gdn_prefill_workspace_bytes_heads(int(total_tokens), int(num_seqs),
                                                     int(heads[0]), int(heads[1])))


def alloc_workspace(total_tokens: int, num_seqs: int, device=None, heads=(H_QK, HV)) -> torch.Tensor:
    """A caller-owned workspace for ``kernel(..., workspace=...)``: uint8 bytes
    sized for any batch of ``total_tokens`` tokens in ``num_seqs`` sequences."""
    dev = torch.device("cuda", torch.cuda.current_device()) if device is None else torch.device(device)
    return torch.empty(max(workspace_bytes(total_tokens, num_seqs, heads), 256),
                       dtype=torch.uint8, device=dev)


def _check_workspace(ws, dev: torch.device, nbytes: int) -> None:
    if not isinstance(ws, torch.Tensor) or ws.dtype != torch.uint8 or ws.dim() != 1:
        raise ValueError("workspace must be a 1-D uint8 tensor (see alloc_workspace)")
    if ws.device != dev:
        raise ValueError(f"workspace is on {ws.device}, expected {dev}")
    if not ws.is_contiguous() or ws.data_ptr() % 256:
        raise ValueError("workspace must be contiguous and 256-byte aligned")
    if ws.numel() < nbytes:
        raise _lib.GdnWorkspaceError(
            f"workspace holds {ws.numel()} bytes; this batch needs {nbytes}")


def _workspace(dev: torch.device, stream: int, nbytes: int) -> torch.Tensor:
    """A byte buffer of at least nbytes, reused by later calls on the same
    stream (work on one stream is ordered, so reuse needs no sync)."""
    key = (dev.index, stream)
    capturing = torch.cuda.is_current_stream_capturing()
    with _ws_lock:
        entry = _workspaces.get(key)
        if entry is None or entry[0].numel() < nbytes:
            if entry is not None and entry[1]:
                _retired.append(entry[0])
            entry = [torch.empty(max(nbytes, 256), dtype=torch.uint8, device=dev), False]
            _workspaces[key] = entry
        if capturing:
            entry[1] = True
        return entry[0]


def release_workspaces() -> int:
    """Drops the cached per-stream workspaces that no captured graph can
    write (torch's caching allocator then owns their memory again); a cached
    buffer a capture has used stays, as it must for the graph's replays.  The
    next call on a stream allocates afresh.  Safe with work still queued: each
    buffer was allocated on its own stream, so the allocator hands its memory
    only to later work on that stream.  Returns the bytes released."""
    freed = 0
    with _ws_lock:
        for key in list(_workspaces):
            buf, captured = _workspaces[key]
            if not captured:
                freed += buf.numel()
                del _workspaces[key]
    return freed


def batch_status(total_tokens: int, num_seqs: int, *, workspace=None, device=None,
                 heads=(H_QK, HV)) -> int:
    """Whether the last prefill call of (T, N) on torch's current stream kept
    the cu_seqlens contract: the OR of the per-sequence status words it left
    in its workspace (gdn_prefill_status_offset, include/gdn_amd.h): 0 for a
    well-formed batch, bit 0 if some cu_seqlens[s+1] < cu_seqlens[s], bit 1 if
    some offset is outside [0, T].  ``workspace`` is the buffer passed to that
    call (default: the stream's cached one).  Synchronises the stream: for
    tests and debugging, not the hot path."""
    lib = _lib.load()
    T, N = int(total_tokens), int(num_seqs)
    if N < 1:
        raise ValueError("a batch without sequences leaves no status")
    dev = torch.device("cuda", torch.cuda.current_device()) if device is None else torch.device(device)
    stream = torch.cuda.current_stream(dev).cuda_stream
    if workspace is None:
        with _ws_lock:
            entry = _workspaces.get((dev.index, stream))
        if entry is None:
            raise ValueError("no prefill call has run on this stream")
        workspace = entry[0]
    need = workspace_bytes(T, N, heads)
    _check_workspace(workspace, dev, need)
    out = ctypes.c_int(0)
    rc = lib.gdn_prefill_status(workspace.data_ptr(), T, N, int(heads[0]), int(heads[1]), stream,
                                ctypes.byref(out))
    _lib.check(rc, "gdn_prefill_status")
    return int(out.value)


def _validate(q, k, v, state, A_log, a, dt_bias, b, cu_seqlens, output, new_state):
    if not isinstance(q, torch.Tensor) or q.dim() != 3:
        raise ValueError("q must be a [T, 4, 128] tensor")
    if not isinstance(v, torch.Tensor) or v.dim() != 3:
        raise ValueError("v must be a [T, 8, 128] tensor")
    T = q.shape[0]
    H_QK, HV = q.shape[1], v.shape[1]
    if H_QK < 1 or HV < 1 or HV % H_QK:
        raise ValueError(f"v-heads ({HV}) must be a multiple of q/k heads ({H_QK})")
    dev = q.device
    if dev.type != "cuda":
        raise ValueError(f"q is on {dev}; the HIP kernels need device tensors")
    if not isinstance(cu_seqlens, torch.Tensor) or cu_seqlens.dim() != 1 or cu_seqlens.numel() < 1:
        raise ValueError("cu_seqlens must be a 1-D tensor of N+1 offsets")
    if cu_seqlens.dtype not in (torch.int32, torch.int64):
        raise ValueError(f"cu_seqlens must be int32 or int64, got {cu_seqlens.dtype}")
    if cu_seqlens.device != dev:
        raise ValueError(f"cu_seqlens is on {cu_seqlens.device}, expected {dev}")
    N = cu_seqlens.numel() - 1
    bf, f32 = torch.bfloat16, torch.float32
    check_tensor("q", q, (T, H_QK, DK), bf, dev)
    check_tensor("k", k, (T, H_QK, DK), bf, dev)
    check_tensor("v", v, (T, HV, DV), bf, dev)
    if state is not None:
        check_tensor("state", state, (N, HV, DV, DK), f32, dev)
    check_tensor("A_log", A_log, (HV,), f32, dev)
    check_tensor("a", a, (T, HV), bf, dev)
    check_tensor("dt_bias", dt_bias, (HV,), f32, dev)
    check_tensor("b", b, (T, HV), bf, dev)
    check_tensor("output", output, (T, HV, DV), bf, dev)
    check_tensor("new_state", new_state, (N, HV, DV, DK), f32, dev)
    check_output("output", output)
    check_output("new_state", new_state)
    return T, N, dev, (H_QK, HV)


def kernel(q, k, v, state, A_log, a, dt_bias, b, cu_seqlens, scale, output, new_state, *,
           variant=-1, workspace=None, recurrent_max_len=-1, recurrent_variant=-1):
    """Chunked GDN prefill over a packed batch, written into ``output`` and
    ``new_state``.

    q, k [T,4,128] bf16; v [T,8,128] bf16; state [N,8,128,128] f32 k-last or
    None; A_log, dt_bias [8] f32; a, b [T,8] bf16; cu_seqlens [N+1] int32/int64
    on the device (monotone, within [0, T]; rows outside [cu[0], cu[N]) get
    zeros); scale float, 0-d tensor or
    None; output [T,8,128] bf16; new_state [N,8,128,128] f32 (may be state).
    ``variant`` picks the form of the per-chunk operands
    (gdn_prefill_fwd_variant): 0 WY, 1 T, -1 the built-in choice; 2 WY with
    one serial chain per sequence, 3 WY with the two-segment scan of a single
    sequence (0 and -1 take it from 9 chunks on), 4 as 3 with the state
    launch's early output of the first half stopped after one chunk per
    workgroup (the output launch then computes the rest: a test of that
    path).  ``workspace``: a caller-owned uint8
    buffer (``alloc_workspace``) used instead of the per-stream cache.
    ``recurrent_max_len``: a batch whose longest sequence has at most this
    many tokens runs through the sequential kernel instead of the chunks (-1
    built-in: token by token, in 16-token blocks or chunks by fitted cost
    models; -2 never);
    ``recurrent_variant``: the sequential kernel (gdn_prefill_fwd_tuned):
    0..9 a token-by-token row tiling, 10 the 16-token block kernel.
    """
    lib = _lib.load()
    T, N, dev, heads = _validate(q, k, v, state, A_log, a, dt_bias, b, cu_seqlens, output,
                                 new_state)
    scale = resolve_scale(scale)
    if state is not None and state.data_ptr() != new_state.data_ptr():
        state = dense(state)
    q, k, v, a, b, A_log, dt_bias, cu_seqlens = (
        dense(t) for t in (q, k, v, a, b, A_log, dt_bias, cu_seqlens))
    stream = stream_of(dev)
    # the kernels store 16 bytes at a time: a view at another offset is
    # computed into an aligned buffer and copied (as the reference's own
    # output.copy_, fla_kernels.py:1052)
    dest = output
    if output.data_ptr() % 16:
        output = torch.empty_like(output)
    nbytes = workspace_bytes(T, N, heads)
    if workspace is None:
        ws = _workspace(dev, stream, nbytes)
    else:
        _check_workspace(workspace, dev, nbytes)
        ws = workspace
    args = (q.data_ptr(), k.data_ptr(), v.data_ptr(), None if state is None else state.data_ptr(),
            A_log.data_ptr(), a.data_ptr(), dt_bias.data_ptr(), b.data_ptr(),
            cu_seqlens.data_ptr(), 1 if cu_seqlens.dtype == torch.int64 else 0, N, T, scale,
            output.data_ptr(), new_state.data_ptr(), ws.data_ptr(), ws.numel(), stream)
    if heads != (H_QK, HV):
        rc = lib.gdn_prefill_fwd_heads(*args[:12], heads[0], heads[1], *args[12:], int(variant),
                                       int(recurrent_max_len), int(recurrent_variant))
    elif recurrent_max_len != -1 or recurrent_variant != -1:
        rc = lib.gdn_prefill_fwd_tuned(*args, int(variant), int(recurrent_max_len),
                                       int(recurrent_variant))
    elif variant == -1:
        rc = lib.gdn_prefill_fwd(*args)
    else:
        rc = lib.gdn_prefill_fwd_variant(*args, int(variant))
    _lib.check(rc, "gdn_prefill_fwd")
    if dest is not output:
        dest.copy_(output)


def run(q, k, v, state, A_log, a, dt_bias, b, cu_seqlens, scale):
    """Non-DPS form with the reference's return convention
    (reference/gdn_prefill_ref.py:12, returns (output, new_state))."""
    T, N = q.shape[0], cu_seqlens.numel() - 1
    HV = v.shape[1]
    output = torch.empty((T, HV, DV), dtype=torch.bfloat16, device=q.device)
    new_state = torch.empty((N, HV, DV, DK), dtype=torch.float32, device=q.device)
    kernel(q, k, v, state, A_log, a, dt_bias, b, cu_seqlens, scale, output, new_state)
    return output, new_state
