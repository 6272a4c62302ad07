"""CPU restatement of the Gated DeltaNet reference operators (numpy).

TEST INFRASTRUCTURE ONLY: imported by ``tests/``, ``__graft_entry__.smoke()``
and the ``cpu_baseline`` leg of ``bench.py`` -- never by the product path.

What each function restates (paths relative to the reference repository):

* :func:`gating`            reference/gdn_decode_ref.py:41-44, gdn_prefill_ref.py:41-44
* :func:`decode`,
  :func:`decode_loop`       reference/gdn_decode_ref.py:26-83
* :func:`prefill_seq`       reference/gdn_prefill_ref.py:26-89
* :func:`chunk_index`       solutions/gdn_prefill_qk4_v8_d128_k_last/solution/triton/
                            fla_kernels.py:58-68 (with the zero-length sequence bug of
                            :63 fixed: seq ids come from the chunk offsets)
* :func:`prefill_chunked`   fla_kernels.py:858-905 (cumsum + beta*K*K^T), 197-314
                            (unit-lower-triangular inverse), 334-383 (w/u), 411-671
                            (inter-chunk state recurrence), 714-796 (chunk output),
                            evaluated in float64 with every mask applied by select.

How each is pinned (the checks live in tests/test_oracle.py; the reference ships
no golden vectors or fixtures for this path):

* gating: float64 closed forms and the limits x>20 -> identity, b->+-inf -> beta
  in {0,1}, A_log->-inf -> decay 1.
* decode: state=0 closed form, beta=0 closed form, delta-overwrite identity
  (|k|=1, beta=1 => S''k = v), GVA head map, and the loop form vs the batched
  form.
* prefill_seq: T=1 equals one decode step; L tokens equal L decode steps;
  split and packing invariance; zero-length sequences give zero state.
* prefill_chunked: equals prefill_seq (an independent algorithm) to ~1e-10 in
  float64; its triangular inverse equals scipy.linalg.solve_triangular.
* chunk_index: brute-force enumeration of chunks.
"""

from __future__ import annotations

import math

import numpy as np

H_QK = 4  # q/k heads        (gdn_decode_ref.py:32-33)
HV = 8  # v heads            (gdn_decode_ref.py:34)
DK = 128  # key head size    (gdn_decode_ref.py:35)
DV = 128  # value head size  (gdn_decode_ref.py:35)
CHUNK = 64  # prefill chunk  (fla_kernels.py:980, BT = 64)
GVA = HV // H_QK


# --------------------------------------------------------------------------
# bf16 helpers (round-to-nearest-even, the rounding torch's .to(bfloat16) uses)
# --------------------------------------------------------------------------

def bf16_bits(x) -> np.ndarray:
    """float32 -> bf16 bit patterns (uint16), round to nearest even, NaN -> 0x7FC0."""
    x = np.ascontiguousarray(np.asarray(x, dtype=np.float32))
    u = x.view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    nan = np.isnan(x)
    if nan.any():
        r = np.where(nan, np.uint16(0x7FC0), r)
    return r


def bf16_from_bits(bits) -> np.ndarray:
    b = np.asarray(bits, dtype=np.uint16).astype(np.uint32) << 16
    return b.view(np.float32)


def bf16_round(x) -> np.ndarray:
    """Round float values to the nearest bf16 value, returned as float32."""
    return bf16_from_bits(bf16_bits(x))


def resolve_scale(scale, head_size: int = DK) -> float:
    """``None`` or ``0.0`` -> 1/sqrt(K); a 0-d array/tensor -> its value.

    Follows reference/gdn_decode_ref.py:38-39 and gdn_prefill_ref.py:38-39.
    """
    if scale is not None and not isinstance(scale, (int, float)):
        scale = float(np.asarray(scale))
    if scale is None or scale == 0.0:
        return 1.0 / math.sqrt(head_size)
    return float(scale)


# --------------------------------------------------------------------------
# gating
# --------------------------------------------------------------------------

def softplus(x):
    """torch.nn.functional.softplus with beta=1, threshold=20: x if x > 20."""
    x = np.asarray(x)
    safe = np.minimum(x, 20.0).astype(x.dtype)
    return np.where(x > 20.0, x, np.log1p(np.exp(safe)))


def log_decay(A_log, a, dt_bias, dtype=np.float32):
    """Log-space decay -exp(A_log) * softplus(a + dt_bias).

    reference/gdn_decode_ref.py:42-43 (the exponent of g); kept in log form as
    the kernels do (solutions/.../triton/kernel.py:49-51).
    """
    x = np.asarray(a, dtype=dtype) + np.asarray(dt_bias, dtype=dtype)
    return (-np.exp(np.asarray(A_log, dtype=dtype)) * softplus(x)).astype(dtype)


def gating(A_log, a, dt_bias, b, dtype=np.float32):
    """(g, beta): g = exp(-exp(A_log)*softplus(a+dt_bias)), beta = sigmoid(b).

    reference/gdn_decode_ref.py:41-44.  ``a`` and ``b`` broadcast against the
    head axis (last) of ``A_log`` / ``dt_bias``.
    """
    g = np.exp(log_decay(A_log, a, dt_bias, dtype)).astype(dtype)
    bb = np.asarray(b, dtype=dtype)
    beta = (1.0 / (1.0 + np.exp(-bb))).astype(dtype)
    return g, beta


# --------------------------------------------------------------------------
# decode
# --------------------------------------------------------------------------

def _expand_heads(x, hv):
    """GVA: v-head h reads q/k head h // (HV / HQK) (repeat_interleave,
    gdn_decode_ref.py:57-58); ``hv`` = number of v-heads."""
    hqk = x.shape[-2]
    assert hv % hqk == 0, "v-heads must be a multiple of q/k heads"
    return np.repeat(x, hv // hqk, axis=-2)


def _heads(q, v):
    """(q/k heads, v-heads) from the tensors: 4 and 8 for the reference
    definitions (gdn_decode_ref.py:32-36); other counts for the generalised
    head configurations, with the same per-head size 128."""
    return q.shape[-2], v.shape[-2]


def decode(q, k, v, state, A_log, a, dt_bias, b, scale, dtype=np.float32):
    """One decode step, batched over (B, HV); op order of gdn_decode_ref.py:72-79.

    q, k: [B,1,4,128]; v: [B,1,8,128]; state: [B,8,128,128] (k-last, [V,K]) or
    None; A_log, dt_bias: [8]; a, b: [B,1,8]. Returns (o [B,1,8,128] as
    bf16-rounded float32, new_state [B,8,128,128] in ``dtype``).  Other head
    counts (HQK q/k heads, HV v-heads, HV a multiple of HQK) follow the shapes.
    """
    B = q.shape[0]
    hqk, HV = _heads(q, v)
    assert q.shape[1:] == (1, hqk, DK) and k.shape[1:] == (1, hqk, DK)
    assert v.shape[1:] == (1, HV, DV)
    scale = resolve_scale(scale)
    g, beta = gating(A_log, a, dt_bias, b, dtype)
    g = g[:, 0]  # [B,HV]
    beta = beta[:, 0]
    qe = _expand_heads(np.asarray(q[:, 0], dtype=dtype), HV)  # [B,HV,K]
    ke = _expand_heads(np.asarray(k[:, 0], dtype=dtype), HV)
    vf = np.asarray(v[:, 0], dtype=dtype)  # [B,HV,V]
    if state is None:
        S = np.zeros((B, HV, DK, DV), dtype=dtype)  # [K,V] view
    else:
        S = np.asarray(state, dtype=dtype).transpose(0, 1, 3, 2)  # [V,K] -> [K,V]
    old_state = g[..., None, None] * S
    old_v = np.matmul(ke[:, :, None, :], old_state)[:, :, 0, :]  # k @ old_state
    new_v = beta[..., None] * vf + (1 - beta[..., None]) * old_v
    state_remove = ke[..., :, None] * old_v[..., None, :]
    state_update = ke[..., :, None] * new_v[..., None, :]
    Snew = old_state - state_remove + state_update
    out = dtype(scale) * np.matmul(qe[:, :, None, :], Snew)[:, :, 0, :]
    o = bf16_round(out.astype(np.float32))[:, None]
    return o, np.ascontiguousarray(Snew.transpose(0, 1, 3, 2))


def decode_loop(q, k, v, state, A_log, a, dt_bias, b, scale):
    """The reference's own loop nest (gdn_decode_ref.py:63-80), one (b, h) at a time.

    Used as the timed CPU baseline; numerically the same op order as decode().
    """
    B = q.shape[0]
    _, HV = _heads(q, v)
    scale = np.float32(resolve_scale(scale))
    g, beta = gating(A_log, a, dt_bias, b)
    qe = _expand_heads(np.asarray(q[:, 0], dtype=np.float32), HV)
    ke = _expand_heads(np.asarray(k[:, 0], dtype=np.float32), HV)
    vf = np.asarray(v[:, 0], dtype=np.float32)
    st = (np.zeros((B, HV, DV, DK), np.float32) if state is None
          else np.asarray(state, dtype=np.float32))
    new_state = np.zeros_like(st)
    output = np.zeros((B, HV, DV), np.float32)
    for bi in range(B):
        for h in range(HV):
            q_h, k_h, v_h = qe[bi, h], ke[bi, h], vf[bi, h]
            h_state = st[bi, h].T.copy()
            gv, bv = g[bi, 0, h], beta[bi, 0, h]
            old_state = gv * h_state
            old_v = k_h @ old_state
            new_v = bv * v_h + (np.float32(1) - bv) * old_v
            h_state = old_state - np.outer(k_h, old_v) + np.outer(k_h, new_v)
            output[bi, h] = scale * (q_h @ h_state)
            new_state[bi, h] = h_state.T
    return bf16_round(output)[:, None], new_state


# --------------------------------------------------------------------------
# prefill: sequential (the reference's algorithm)
# --------------------------------------------------------------------------

def _check_prefill_shapes(q, k, v, a, b, cu_seqlens):
    T = q.shape[0]
    hqk, hv = _heads(q, v)
    assert q.shape == (T, hqk, DK) and k.shape == (T, hqk, DK)
    assert v.shape == (T, hv, DV) and hv % hqk == 0
    assert a.shape == (T, hv) and b.shape == (T, hv)
    cu = np.asarray(cu_seqlens, dtype=np.int64)
    assert cu.ndim == 1 and cu.size >= 1
    return T, cu


def prefill_seq(q, k, v, state, A_log, a, dt_bias, b, cu_seqlens, scale,
                dtype=np.float32):
    """Token-by-token prefill, vectorised over heads (gdn_prefill_ref.py:56-89).

    q, k: [T,4,128]; v: [T,8,128]; a, b: [T,8]; state: [N,8,128,128] or None;
    cu_seqlens: [N+1].  Returns (o [T,8,128] bf16-rounded float32 -- rounded per
    token as gdn_prefill_ref.py:87 does -- and new_state [N,8,128,128]).
    A zero-length sequence leaves its new_state at zero (gdn_prefill_ref.py:61-62).
    """
    T, cu = _check_prefill_shapes(q, k, v, a, b, cu_seqlens)
    N = cu.size - 1
    _, HV = _heads(q, v)
    scale = dtype(resolve_scale(scale))
    g, beta = gating(A_log, a, dt_bias, b, dtype)  # [T,HV]
    qe = _expand_heads(np.asarray(q, dtype=dtype), HV)
    ke = _expand_heads(np.asarray(k, dtype=dtype), HV)
    vf = np.asarray(v, dtype=dtype)
    out = np.zeros((T, HV, DV), np.float32)
    new_state = np.zeros((N, HV, DV, DK), dtype)
    one = dtype(1)
    for s in range(N):
        bos, eos = int(cu[s]), int(cu[s + 1])
        if eos - bos <= 0:
            continue
        if state is not None:
            S = np.asarray(state[s], dtype=dtype).transpose(0, 2, 1).copy()  # [HV,K,V]
        else:
            S = np.zeros((HV, DK, DV), dtype)
        for t in range(bos, eos):
            gt = g[t][:, None, None]
            bt = beta[t][:, None]
            old = gt * S
            old_v = np.matmul(ke[t][:, None, :], old)[:, 0, :]
            new_v = bt * vf[t] + (one - bt) * old_v
            S = old - ke[t][:, :, None] * old_v[:, None, :] + ke[t][:, :, None] * new_v[:, None, :]
            o = scale * np.matmul(qe[t][:, None, :], S)[:, 0, :]
            out[t] = bf16_round(o.astype(np.float32))
        new_state[s] = S.transpose(0, 2, 1)
    return out, new_state


# --------------------------------------------------------------------------
# prefill: chunk index (integer work)
# --------------------------------------------------------------------------

def chunk_index(cu_seqlens, chunk: int = CHUNK):
    """Chunk table for a packed batch.

    Returns (chunk_seq [NT], chunk_local [NT], chunk_offsets [N+1]) where chunk
    c belongs to sequence chunk_seq[c], is its chunk_local[c]-th chunk and
    chunk_offsets is the exclusive prefix sum of ceil(len/64)
    (fla_kernels.py:58-68).  Unlike fla_kernels.py:63, the sequence id is taken
    from the offsets, so a zero-length sequence does not shift later ids.
    """
    cu = np.asarray(cu_seqlens, dtype=np.int64)
    lens = np.diff(cu)
    if (lens < 0).any():
        raise ValueError("cu_seqlens must be non-decreasing")
    n = (lens + chunk - 1) // chunk
    offsets = np.concatenate([[0], np.cumsum(n)]).astype(np.int64)
    seq = np.repeat(np.arange(lens.size, dtype=np.int64), n)
    local = np.arange(offsets[-1], dtype=np.int64) - offsets[seq]
    return seq, local, offsets


def max_chunks(total_tokens: int, num_seqs: int, chunk: int = CHUNK) -> int:
    """Upper bound on the chunk count that needs no look at cu_seqlens.

    sum_i ceil(L_i/C) <= sum_i (L_i + C - 1)/C = (T + N(C-1))/C, and it is also
    at most T (every chunk holds >= 1 token).
    """
    if total_tokens <= 0 or num_seqs <= 0:
        return 0
    return min(total_tokens, (total_tokens + num_seqs * (chunk - 1)) // chunk)


# --------------------------------------------------------------------------
# prefill: chunked WY form (float64), exposing the intermediates
# --------------------------------------------------------------------------

def prefill_chunked(q, k, v, state, A_log, a, dt_bias, b, cu_seqlens, scale,
                    return_intermediates: bool = False):
    """Chunk-64 WY evaluation of the prefill in float64.

    Per sequence, v-head and chunk (C <= 64 rows; G = chunk-local cumsum of the
    log decay, g_i = log-decay of token i, beta_i = sigmoid(b_i)):

    * G      = cumsum(g)                                  fla_kernels.py:884-890
    * A_ij   = beta_i exp(G_i - G_j) <k_i,k_j>  (i > j)   fla_kernels.py:893-905
    * Ai     = (I + A)^-1                                  fla_kernels.py:197-314
    * u      = Ai (beta * V),  w = Ai (beta exp(G) * K)    fla_kernels.py:361-383
    * h      = S  (state at chunk start, [K,V])            fla_kernels.py:505-528
    * v_new  = u - w S                                     fla_kernels.py:530-560
    * o_i    = scale (exp(G_i) q_i S
               + sum_{j<=i} exp(G_i-G_j) <q_i,k_j> v_new_j) fla_kernels.py:755-796
    * S     <- exp(G_last) S + K^T (exp(G_last - G) * v_new) fla_kernels.py:566-645

    Returns (o [T,8,128] float64 -- not rounded --, new_state [N,8,128,128]
    float64) and, if asked, a dict of per-chunk intermediates keyed by name
    with arrays indexed [chunk, head, ...] in chunk_index() order.
    """
    T, cu = _check_prefill_shapes(q, k, v, a, b, cu_seqlens)
    N = cu.size - 1
    _, HV = _heads(q, v)
    f = np.float64
    scale = resolve_scale(scale)
    glog = log_decay(A_log, a, dt_bias, f)  # [T,HV]
    beta = 1.0 / (1.0 + np.exp(-np.asarray(b, f)))
    qe = _expand_heads(np.asarray(q, f), HV)
    ke = _expand_heads(np.asarray(k, f), HV)
    vf = np.asarray(v, f)
    out = np.zeros((T, HV, DV), f)
    new_state = np.zeros((N, HV, DV, DK), f)
    seq_of, local_of, offs = chunk_index(cu)
    NT = int(offs[-1])
    inter = None
    if return_intermediates:
        inter = {
            "g_cs": np.zeros((NT, HV, CHUNK), f),
            "A": np.zeros((NT, HV, CHUNK, CHUNK), f),
            "Ai": np.zeros((NT, HV, CHUNK, CHUNK), f),
            "w": np.zeros((NT, HV, CHUNK, DK), f),
            "u": np.zeros((NT, HV, CHUNK, DV), f),
            "h": np.zeros((NT, HV, DK, DV), f),
            "v_new": np.zeros((NT, HV, CHUNK, DV), f),
        }
    for s in range(N):
        bos, eos = int(cu[s]), int(cu[s + 1])
        L = eos - bos
        if L <= 0:
            continue
        for h in range(HV):
            if state is not None:
                S = np.asarray(state[s, h], f).T.copy()  # [K,V]
            else:
                S = np.zeros((DK, DV), f)
            for c in range((L + CHUNK - 1) // CHUNK):
                t0 = bos + c * CHUNK
                t1 = min(t0 + CHUNK, eos)
                C = t1 - t0
                G = np.cumsum(glog[t0:t1, h])
                Kc, Qc, Vc = ke[t0:t1, h], qe[t0:t1, h], vf[t0:t1, h]
                bc = beta[t0:t1, h]
                ii, jj = np.meshgrid(np.arange(C), np.arange(C), indexing="ij")
                dG = np.where(ii >= jj, G[:, None] - G[None, :], -np.inf)
                decay_ij = np.exp(dG)  # 0 above the diagonal, by select
                A = np.where(ii > jj, bc[:, None] * decay_ij * (Kc @ Kc.T), 0.0)
                Ai = np.linalg.inv(np.eye(C) + A)
                u = Ai @ (bc[:, None] * Vc)
                w = Ai @ ((bc * np.exp(G))[:, None] * Kc)
                h_start = S.copy()
                v_new = u - w @ S
                attn = np.where(ii >= jj, decay_ij * (Qc @ Kc.T), 0.0)
                o = scale * (np.exp(G)[:, None] * (Qc @ S) + attn @ v_new)
                out[t0:t1, h] = o
                S = np.exp(G[-1]) * S + Kc.T @ (np.exp(G[-1] - G)[:, None] * v_new)
                if inter is not None:
                    ci = int(offs[s]) + c
                    inter["g_cs"][ci, h, :C] = G
                    inter["A"][ci, h, :C, :C] = A
                    inter["Ai"][ci, h, :C, :C] = Ai
                    inter["w"][ci, h, :C] = w
                    inter["u"][ci, h, :C] = u
                    inter["h"][ci, h] = h_start
                    inter["v_new"][ci, h, :C] = v_new
            new_state[s, h] = S.T
    if return_intermediates:
        return out, new_state, inter
    return out, new_state


# --------------------------------------------------------------------------
# seeded synthetic inputs (the recipe of BASELINE.json configs 0-4)
# --------------------------------------------------------------------------

def _l2norm_bf16(x):
    x = x / np.linalg.norm(x, axis=-1, keepdims=True)
    return bf16_round(x.astype(np.float32))


def make_decode_inputs(B: int, seed: int = 0, with_state: bool = True, heads=(H_QK, HV)):
    """Decode inputs of configs[0]/[1]: numpy default_rng(seed), draw order
    q, k, v, state, A_log, a, dt_bias, b; q/k L2-normalised per head then
    rounded to bf16; state ~ N(0, 0.05^2) (0.05 read as the std. deviation).
    ``heads`` = (q/k heads, v-heads), (4, 8) for the reference definitions."""
    H_QK, HV = heads
    rng = np.random.default_rng(seed)
    q = _l2norm_bf16(rng.standard_normal((B, 1, H_QK, DK)))
    k = _l2norm_bf16(rng.standard_normal((B, 1, H_QK, DK)))
    v = bf16_round(rng.standard_normal((B, 1, HV, DV)).astype(np.float32))
    state = (0.05 * rng.standard_normal((B, HV, DV, DK))).astype(np.float32)
    A_log = rng.uniform(0.0, math.log(16.0), HV).astype(np.float32)
    a = bf16_round(rng.standard_normal((B, 1, HV)).astype(np.float32))
    dt_bias = rng.uniform(0.0, 1.0, HV).astype(np.float32)
    b = bf16_round(rng.standard_normal((B, 1, HV)).astype(np.float32))
    return dict(q=q, k=k, v=v, state=state if with_state else None, A_log=A_log,
                a=a, dt_bias=dt_bias, b=b, scale=1.0 / math.sqrt(DK))


def make_prefill_inputs(lens, seed: int = 0, with_state: bool = True,
                        slow_decay_heads=(), heads=(H_QK, HV)):
    """Prefill inputs of configs[2]-[4] (same recipe as make_decode_inputs).

    ``slow_decay_heads`` get A_log = -10 (decay ~ 1 - 5e-5 per token), the
    skew configs[4] asks for.  Returns the tensors plus cu_seqlens (int64).
    """
    H_QK, HV = heads
    lens = [int(x) for x in lens]
    T = sum(lens)
    N = len(lens)
    rng = np.random.default_rng(seed)
    q = _l2norm_bf16(rng.standard_normal((T, H_QK, DK)))
    k = _l2norm_bf16(rng.standard_normal((T, H_QK, DK)))
    v = bf16_round(rng.standard_normal((T, HV, DV)).astype(np.float32))
    state = (0.05 * rng.standard_normal((N, HV, DV, DK))).astype(np.float32)
    A_log = rng.uniform(0.0, math.log(16.0), HV).astype(np.float32)
    for h in slow_decay_heads:
        A_log[h] = -10.0
    a = bf16_round(rng.standard_normal((T, HV)).astype(np.float32))
    dt_bias = rng.uniform(0.0, 1.0, HV).astype(np.float32)
    b = bf16_round(rng.standard_normal((T, HV)).astype(np.float32))
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int64)
    return dict(q=q, k=k, v=v, state=state if with_state else None, A_log=A_log,
                a=a, dt_bias=dt_bias, b=b, cu_seqlens=cu, scale=1.0 / math.sqrt(DK))


def make_all_same_inputs(lens, value: float = 0.5, noise: float = 0.0, seed: int = 0,
                         with_state: bool = True):
    """The reference's "all_same" adversarial input (OPTIMIZATION_LOG.md:217-220):
    every tensor -- q, k, v, state, A_log, a, dt_bias, b -- filled with
    ``value``; scale 1/sqrt(128).  With 0.5, beta |k|^2 = 19.9 and the decay
    is 0.115, so the state grows ~2.2x per token (f32 stays finite to ~110
    tokens).  ``noise`` > 0 multiplies each element by (1 + noise N(0,1)) so
    the tensors are no longer uniform.  Returns prefill inputs for ``lens``
    (cu_seqlens int64); bf16 tensors are rounded to bf16."""
    lens = [int(x) for x in lens]
    T, N = sum(lens), len(lens)
    rng = np.random.default_rng(seed)

    def fill(shape, bf16=True):
        x = np.full(shape, value, np.float32)
        if noise:
            x = (x * (1.0 + noise * rng.standard_normal(shape))).astype(np.float32)
        return bf16_round(x) if bf16 else x

    q, k, v = fill((T, H_QK, DK)), fill((T, H_QK, DK)), fill((T, HV, DV))
    state = fill((N, HV, DV, DK), bf16=False)
    A_log, a, dt_bias, b = fill((HV,), False), fill((T, HV)), fill((HV,), False), fill((T, HV))
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int64)
    return dict(q=q, k=k, v=v, state=state if with_state else None, A_log=A_log, a=a,
                dt_bias=dt_bias, b=b, cu_seqlens=cu, scale=1.0 / math.sqrt(DK))


# The workloads of BASELINE.json, in one place.
CONFIGS = {
    "decode_b1": dict(kind="decode", B=1, seed=0),
    "decode_sweep": dict(kind="decode", Bs=(1, 2, 4, 8, 16, 32, 48, 64), seed=1),
    "prefill_1x1024": dict(kind="prefill", lens=(1024,), seed=2, with_state=False),
    "prefill_varlen6": dict(kind="prefill", lens=(6, 49, 294, 1800, 2040, 61), seed=3,
                            with_state=True),
    "prefill_4x8192": dict(kind="prefill", lens=(8192,) * 4, seed=4, with_state=True,
                           slow_decay_heads=(6, 7)),
    "prefill_1x8192": dict(kind="prefill", lens=(8192,), seed=2, with_state=False),
}


# --------------------------------------------------------------------------
# algorithmic work (bytes / flops) per launch
# --------------------------------------------------------------------------

def decode_bytes(B: int) -> int:
    """Compulsory HBM bytes of one decode step: state in + out (f32), q, k, v,
    o (bf16), a, b (bf16) per batch row, plus A_log and dt_bias."""
    per_b = 2 * HV * DV * DK * 4 + 2 * H_QK * DK * 2 + HV * DV * 2 + 2 * HV * 2 + HV * DV * 2
    return per_b * B + 2 * HV * 4


def decode_flops(B: int) -> int:
    """7 flops per state element: decay 1, S.k 2, rank-1 update 2, S.q 2."""
    return 7 * HV * DV * DK * B


def prefill_bytes(T: int, N: int) -> int:
    """Compulsory HBM bytes of one prefill: q, k (4 heads) and v, o (8 heads)
    in bf16, a and b in bf16, the initial and final state (f32), cu_seqlens
    and A_log / dt_bias."""
    return (T * (2 * H_QK * DK * 2 + 2 * HV * DV * 2 + 2 * HV * 2)
            + N * 2 * HV * DV * DK * 4 + 8 * (N + 1) + 2 * HV * 4)


def prefill_flops(NT: int) -> int:
    """11 units of 2*64*128*64 flops per (chunk, head): K K^T 1, w 1, u 1,
    w S 2, K^T v_new 2, Q S 2, Q K^T 1, (QK^T) v_new 1."""
    return NT * HV * 11 * 2 * CHUNK * DK * CHUNK


# --------------------------------------------------------------------------
# C restatement of the sequential recurrence (oracle/gdn_seq.c), for full sizes
# --------------------------------------------------------------------------

_CLIB = None


def _clib():
    global _CLIB
    if _CLIB is None:
        import ctypes
        import os
        path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libgdn_oracle.so")
        if not os.path.exists(path):
            raise RuntimeError(f"C oracle not built: {path} (run `make -C oracle`)")
        lib = ctypes.CDLL(path)
        P = ctypes.c_void_p
        lib.gdn_oracle_prefill_seq.argtypes = [P, P, P, P, P, P, P, ctypes.c_int,
                                               ctypes.c_int, ctypes.c_int, ctypes.c_float,
                                               P, P, ctypes.c_int]
        lib.gdn_oracle_prefill_seq.restype = ctypes.c_int
        lib.gdn_oracle_set_threads.argtypes = [ctypes.c_int]
        lib.gdn_oracle_set_threads.restype = ctypes.c_int
        _CLIB = lib
    return _CLIB


def set_c_threads(n: int) -> int:
    """OpenMP threads of prefill_seq_c's (sequence, v-head) loop for later
    calls from this thread (n <= 0: every processor); returns the count."""
    return int(_clib().gdn_oracle_set_threads(int(n)))


def prefill_seq_c(q, k, v, state, A_log, a, dt_bias, b, cu_seqlens, scale,
                  use_f64: bool = False):
    """prefill_seq() through the C recurrence: same algorithm and op order
    (gdn_prefill_ref.py:71-89), OpenMP over (sequence, head).  Gating is the
    numpy float32 gating() above.  Returns (o bf16-rounded float32, new_state)."""
    T, cu = _check_prefill_shapes(q, k, v, a, b, cu_seqlens)
    N = cu.size - 1
    hqk, HV = _heads(q, v)
    g, beta = gating(A_log, a, dt_bias, b, np.float32)
    arrs = [np.ascontiguousarray(x, dtype=np.float32) for x in (q, k, v, g, beta)]
    st = None if state is None else np.ascontiguousarray(state, dtype=np.float32)
    cu = np.ascontiguousarray(cu, dtype=np.int64)
    o = np.zeros((T, HV, DV), np.float32)
    ns = np.zeros((N, HV, DV, DK), np.float32)
    ptr = lambda x: None if x is None else x.ctypes.data
    rc = _clib().gdn_oracle_prefill_seq(*[ptr(x) for x in arrs], ptr(st), ptr(cu), N, hqk, HV,
                                        float(resolve_scale(scale)), ptr(o), ptr(ns),
                                        1 if use_f64 else 0)
    if rc != 0:
        raise ValueError("gdn_oracle_prefill_seq rejected its arguments")
    return bf16_round(o), ns
