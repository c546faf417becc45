"""CPU oracle for ``masked_attention_via_map`` -- TEST INFRASTRUCTURE ONLY.

This module is the checker, never the product.  Only ``tests/``,
``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` may
import it.  The shipped code path (``jaxmodules_amd``) must never call into it.

It restates, in plain numpy, the semantics of the reference's masked attention
(``/root/reference/jaxmodules/attention.py``):

* ``canonical_plan``      -- argument validation, mask canonicalisation,
  padding and the block-granular, clamped ``window_size`` rule
  (attention.py:195-217, 161-167, 385-437).
* ``effective_mask``      -- the dense boolean mask [B, Hq, N, L] the reference
  actually applies: ``mask_fn`` AND window-visited key blocks.
* ``dense_forward`` / ``dense_backward`` -- float64 closed-form masked softmax
  attention and its analytic gradients (the maths the reference computes,
  attention.py:52-105 and the custom_vjp at :266-342).  Rows with no allowed
  key give O = 0 and zero gradients (attention.py:93-100).
* ``blockwise_forward`` / ``blockwise_backward`` -- a loop-for-loop
  restatement of the reference's *algorithm* (lax.map over query blocks,
  scan over every visited key block, dense per-tile mask, unnormalised
  ``exp`` running average, per-query-block recompute in the backward pass).
  Used as the CPU baseline and pinned against ``dense_*``.

Pinning (see tests/test_oracle.py): the dense functions are checked against
torch's scaled_dot_product_attention and torch autograd (an independent
implementation, as the reference's own tests do, test_mapped_attention.py:31-300),
against closed forms (uniform attention, zero inputs, fully-masked rows), and
the window rule against the reference tests' relations
(test_mapped_attention.py:1552-1648, 1762-1798).
"""
from __future__ import annotations

import math
from dataclasses import dataclass
from typing import Callable, Optional, Tuple

import numpy as np


# --------------------------------------------------------------------------
# argument canonicalisation (attention.py:385-437 and :195-217)
# --------------------------------------------------------------------------


@dataclass
class Plan:
    B: int
    N: int
    L: int
    Hq: int
    Hkv: int
    d: int
    bs: int            # query block size == key block size (attention.py:155)
    Npad: int          # padded query length
    Lpad: int          # padded key length
    mask4: Callable    # canonical 4-argument mask_fn (b, h, q, k)
    window: Optional[Tuple[int, int]]  # (left_blocks, right_blocks) or None
    squeeze_batch: bool


def _canonical_mask(is_causal, mask_fn):
    """attention.py:404-419."""
    if mask_fn is not None and mask_fn.__code__.co_argcount == 3:
        three = mask_fn
        mask_fn = lambda b, h, q, k: three(h, q, k)  # noqa: E731
    if is_causal and mask_fn is not None:
        raise ValueError("cannot specify both 'is_causal' and 'mask_fn'!")
    if is_causal:
        mask_fn = lambda b, h, q, k: q >= k  # noqa: E731
    if mask_fn is None:
        mask_fn = lambda b, h, q, k: True  # noqa: E731
    return mask_fn


def canonical_plan(q_shape, k_shape, v_shape, *, is_causal=False, mask_fn=None,
                   block_size=None, window_size=None) -> Plan:
    """Restates the reference's validation and set-up.

    attention.py:385-391 (ndim -> ValueError), :394-399 (3D -> batch dim),
    :404-419 (mask canonicalisation), :421-437 (padding), :195-217 (block size,
    window blocks, shape asserts -> AssertionError), :155 (key blocks use the
    query block size, so L must split into blocks of bs).
    """
    for name, s in (("K", k_shape), ("Q", q_shape), ("V", v_shape)):
        if len(s) not in (3, 4):
            raise ValueError(f"{name} must have 3 or 4 dimensions")
    assert len(k_shape) == len(q_shape) and len(v_shape) == len(q_shape)
    squeeze = len(q_shape) == 3
    if squeeze:
        q_shape, k_shape, v_shape = (1,) + tuple(q_shape), (1,) + tuple(k_shape), (1,) + tuple(v_shape)
    mask4 = _canonical_mask(is_causal, mask_fn)
    assert k_shape[0] == q_shape[0] == v_shape[0]
    B, N, Hq, dq = q_shape
    _, L, Hk, d = k_shape
    _, Lv, Hv, dv = v_shape
    Npad, Lpad = N, L
    if block_size is not None and N % block_size != 0:
        Npad = N + block_size - N % block_size
        Lpad = L + block_size - L % block_size      # a whole extra block when L % bs == 0
    bs = Npad if block_size is None else block_size
    assert d == dq and Lv == L and dv == d, "shape mismatch"
    assert Hq % Hk == 0, "Hq must be divisible by Hk"
    assert Hv == Hk, "Hv must be equal to Hk"
    if Lpad % bs != 0:
        # einops rearrange "B (blocks block_size) ..." fails in the reference
        raise RuntimeError(f"key length {Lpad} is not a multiple of the block size {bs}")
    window = None
    if window_size is not None:
        left, right = window_size
        lwb = (left + bs - 1) // bs
        rwb = 1 + (right + bs - 1) // bs
        window = (lwb, rwb)
        if lwb + rwb > Lpad // bs:
            # lax.dynamic_slice_in_dim rejects a slice larger than the operand
            raise TypeError("window covers more key blocks than exist")
    return Plan(B, N, L, Hq, Hk, d, bs, Npad, Lpad, mask4, window, squeeze)


def visited_key_blocks(i: int, nk: int, window) -> range:
    """Key blocks the reference scans for query block ``i`` (attention.py:160-167).

    ``lax.dynamic_slice_in_dim`` clamps its start index into ``[0, nk - size]``.
    """
    if window is None:
        return range(nk)
    lwb, rwb = window
    total = lwb + rwb
    start = max(0, i - lwb)
    start = min(start, nk - total)
    return range(start, start + total)


def _eval_mask(mask4, b, h, q, k):
    """Elementwise evaluation of a 4-argument mask on broadcast index arrays
    (the reference evaluates it under nested vmaps, vectorize.py:407-527)."""
    m = mask4(b, h, q, k)
    shape = np.broadcast_shapes(np.shape(b), np.shape(h), np.shape(q), np.shape(k))
    return np.broadcast_to(np.asarray(m, dtype=bool), shape)


def effective_mask(plan: Plan) -> np.ndarray:
    """Dense [B, Hq, N, L] boolean mask the reference applies (unpadded range)."""
    B, Hq, N, L = plan.B, plan.Hq, plan.N, plan.L
    b = np.arange(B, dtype=np.int64)[:, None, None, None]
    h = np.arange(Hq, dtype=np.int64)[None, :, None, None]
    q = np.arange(N, dtype=np.int64)[None, None, :, None]
    k = np.arange(L, dtype=np.int64)[None, None, None, :]
    m = _eval_mask(plan.mask4, b, h, q, k).copy()
    if plan.window is not None:
        nq, nk = plan.Npad // plan.bs, plan.Lpad // plan.bs
        vis = np.zeros((nq, nk), dtype=bool)
        for i in range(nq):
            vis[i, list(visited_key_blocks(i, nk, plan.window))] = True
        qb = np.arange(N) // plan.bs
        kb = np.arange(L) // plan.bs
        m &= vis[qb][:, kb][None, None]
    return m


# --------------------------------------------------------------------------
# float64 dense closed form
# --------------------------------------------------------------------------


def _expand_kv(X, Hq):
    """GQA: query head h reads key/value head h // (Hq / Hkv) (attention.py:66-68)."""
    G = Hq // X.shape[2]
    return np.repeat(X, G, axis=2)


def dense_forward(Q, K, V, allowed, scale=None):
    """O [B,N,Hq,d] and natural-log LSE [B,Hq,N] (-inf for empty rows), float64."""
    Q = np.asarray(Q, np.float64)
    K = np.asarray(K, np.float64)
    V = np.asarray(V, np.float64)
    B, N, Hq, d = Q.shape
    scale = 1.0 / math.sqrt(d) if scale is None else scale
    Kx, Vx = _expand_kv(K, Hq), _expand_kv(V, Hq)
    S = np.einsum("bqhd,bkhd->bhqk", Q, Kx) * scale
    S = np.where(allowed, S, -np.inf)
    m = S.max(axis=-1, keepdims=True)
    m = np.where(np.isfinite(m), m, 0.0)
    P = np.where(allowed, np.exp(S - m), 0.0)
    l = P.sum(axis=-1, keepdims=True)
    Pn = P / np.where(l > 0, l, 1.0)
    O = np.einsum("bhqk,bkhd->bqhd", Pn, Vx)
    with np.errstate(divide="ignore"):
        lse = np.where(l[..., 0] > 0, m[..., 0] + np.log(l[..., 0]), -np.inf)
    return O, lse


def dense_probs_ds(Q, K, V, allowed, dO, scale=None):
    """(P, dS) [B,Hq,N,L] float64: the normalised attention weights and the
    score gradient dS = P (dP - delta), dP = dO V^T, delta = rowsum(dP * P)
    (attention.py:266-342's per-tile quantities, over the whole matrix)."""
    Q = np.asarray(Q, np.float64)
    K = np.asarray(K, np.float64)
    V = np.asarray(V, np.float64)
    dO = np.asarray(dO, np.float64)
    Hq, d = Q.shape[2], Q.shape[3]
    scale = 1.0 / math.sqrt(d) if scale is None else scale
    Kx, Vx = _expand_kv(K, Hq), _expand_kv(V, Hq)
    S = np.einsum("bqhd,bkhd->bhqk", Q, Kx) * scale
    S = np.where(allowed, S, -np.inf)
    m = S.max(axis=-1, keepdims=True)
    m = np.where(np.isfinite(m), m, 0.0)
    P = np.where(allowed, np.exp(S - m), 0.0)
    l = P.sum(axis=-1, keepdims=True)
    P = P / np.where(l > 0, l, 1.0)
    dP = np.einsum("bqhd,bkhd->bhqk", dO, Vx)
    delta = (dP * P).sum(axis=-1, keepdims=True)      # == rowsum(dO * O)
    return P, P * (dP - delta)


def dense_backward(Q, K, V, allowed, dO, scale=None):
    """Analytic gradients of sum(O * dO) w.r.t. Q, K, V, float64."""
    Q = np.asarray(Q, np.float64)
    K = np.asarray(K, np.float64)
    dO = np.asarray(dO, np.float64)
    B, N, Hq, d = Q.shape
    Hkv = K.shape[2]
    G = Hq // Hkv
    scale = 1.0 / math.sqrt(d) if scale is None else scale
    Kx = _expand_kv(K, Hq)
    P, dS = dense_probs_ds(Q, K, V, allowed, dO, scale)
    dQ = np.einsum("bhqk,bkhd->bqhd", dS, Kx) * scale
    dKx = np.einsum("bhqk,bqhd->bkhd", dS, Q) * scale
    dVx = np.einsum("bhqk,bqhd->bkhd", P, dO)
    Bk, L = K.shape[0], K.shape[1]
    dK = dKx.reshape(Bk, L, Hkv, G, d).sum(axis=3)
    dV = dVx.reshape(Bk, L, Hkv, G, d).sum(axis=3)
    return dQ, dK, dV


def reference_attention(Q, K, V, *, is_causal=False, mask_fn=None, block_size=None,
                        window_size=None):
    """Full drop-in semantics, float64: returns O (same rank as Q)."""
    plan = canonical_plan(Q.shape, K.shape, V.shape, is_causal=is_causal, mask_fn=mask_fn,
                          block_size=block_size, window_size=window_size)
    if plan.squeeze_batch:
        Q, K, V = Q[None], K[None], V[None]
    O, _ = dense_forward(Q, K, V, effective_mask(plan))
    return O[0] if plan.squeeze_batch else O


def reference_attention_grads(Q, K, V, dO, *, is_causal=False, mask_fn=None,
                              block_size=None, window_size=None):
    plan = canonical_plan(Q.shape, K.shape, V.shape, is_causal=is_causal, mask_fn=mask_fn,
                          block_size=block_size, window_size=window_size)
    if plan.squeeze_batch:
        Q, K, V, dO = Q[None], K[None], V[None], dO[None]
    g = dense_backward(Q, K, V, effective_mask(plan), dO)
    return tuple(x[0] for x in g) if plan.squeeze_batch else g


# --------------------------------------------------------------------------
# blockwise restatement of the reference algorithm (CPU baseline)
# --------------------------------------------------------------------------


def _tile_mask(plan: Plan, b_idx, q_idx, k_idx):
    """Per-tile mask [B, Hq, bq, bk] exactly as the reference evaluates it: the
    canonical mask on padded indices, AND (q<N)&(k<L) when padded (attention.py:437)."""
    b = b_idx[:, None, None, None]
    h = np.arange(plan.Hq)[None, :, None, None]
    q = q_idx[None, None, :, None]
    k = k_idx[None, None, None, :]
    m = _eval_mask(plan.mask4, b, h, q, k)
    if plan.Npad != plan.N or plan.Lpad != plan.L:
        m = m & (q < plan.N) & (k < plan.L)
    return m


def blockwise_forward(Q, K, V, plan: Plan, dtype=np.float32, q_blocks=None):
    """attention.py:133-241: for each query block, scan every visited key block
    with the unnormalised kernel exp(q.k/sqrt(d)), the dense tile mask and the
    running-average update of :91-100.  No tile is skipped.

    Q/K/V are [B, Npad|N, H, d] arrays (padding applied by the caller if needed).
    ``q_blocks`` restricts the work to a subset of query blocks (baseline sampling).
    Returns O [B, Npad, Hq, d] (rows of skipped blocks are zero).
    """
    B, Nq, Hq, d = Q.shape
    Hkv = K.shape[2]
    G = Hq // Hkv
    bs = plan.bs
    nq, nk = plan.Npad // bs, plan.Lpad // bs
    Qp = np.zeros((B, plan.Npad, Hq, d), dtype)
    Qp[:, :Nq] = Q
    Kp = np.zeros((B, plan.Lpad, Hkv, d), dtype)
    Kp[:, :K.shape[1]] = K
    Vp = np.zeros((B, plan.Lpad, Hkv, d), dtype)
    Vp[:, :V.shape[1]] = V
    # heads-major copies so matmul runs on contiguous [.., rows, d] matrices
    Qh = np.ascontiguousarray(Qp.transpose(0, 2, 1, 3))            # [B,Hq,Npad,d]
    Kh = np.ascontiguousarray(np.repeat(Kp, G, axis=2).transpose(0, 2, 3, 1))  # [B,Hq,d,Lpad]
    Vh = np.ascontiguousarray(np.repeat(Vp, G, axis=2).transpose(0, 2, 1, 3))  # [B,Hq,Lpad,d]
    inv = dtype(1.0 / math.sqrt(d))
    out = np.zeros((B, Hq, plan.Npad, d), dtype)
    bidx = np.arange(B)
    for i in (range(nq) if q_blocks is None else q_blocks):
        qs = slice(i * bs, (i + 1) * bs)
        q_idx = np.arange(i * bs, (i + 1) * bs)
        Z = np.zeros((B, Hq, bs, 1), dtype)
        O = np.zeros((B, Hq, bs, d), dtype)
        for j in visited_key_blocks(i, nk, plan.window):
            ks = slice(j * bs, (j + 1) * bs)
            k_idx = np.arange(j * bs, (j + 1) * bs)
            sc = np.exp(np.matmul(Qh[:, :, qs], Kh[:, :, :, ks]) * inv)
            sc *= _tile_mask(plan, bidx, q_idx, k_idx)
            loc = sc.sum(axis=-1, keepdims=True)
            u = np.matmul(sc, Vh[:, :, ks])
            Zn = Z + loc
            safe = np.where(Zn > 0, Zn, 1)
            O = np.where(Zn > 0, O + (u - O * loc) / safe, 0)
            Z = Zn
        out[:, :, qs] = O
    return out.transpose(0, 2, 1, 3)


def blockwise_backward(Q, K, V, dO, plan: Plan, dtype=np.float32, q_blocks=None):
    """attention.py:266-342: a scan over query blocks; each block recomputes its
    whole key scan and back-propagates through it (jax.vjp of _attn_block_fn),
    producing dq for the block and full-size dK/dV contributions that are added
    into carries.  The per-block vjp is written out analytically here.
    """
    B, Nq, Hq, d = Q.shape
    Hkv = K.shape[2]
    G = Hq // Hkv
    bs = plan.bs
    nq, nk = plan.Npad // bs, plan.Lpad // bs
    Qp = np.zeros((B, plan.Npad, Hq, d), dtype)
    Qp[:, :Nq] = Q
    dOp = np.zeros((B, plan.Npad, Hq, d), dtype)
    dOp[:, :Nq] = dO
    Kp = np.zeros((B, plan.Lpad, Hkv, d), dtype)
    Kp[:, :K.shape[1]] = K
    Vp = np.zeros((B, plan.Lpad, Hkv, d), dtype)
    Vp[:, :V.shape[1]] = V
    Qh = np.ascontiguousarray(Qp.transpose(0, 2, 1, 3))
    dOh = np.ascontiguousarray(dOp.transpose(0, 2, 1, 3))
    Kh = np.ascontiguousarray(np.repeat(Kp, G, axis=2).transpose(0, 2, 1, 3))   # [B,Hq,Lpad,d]
    Vh = np.ascontiguousarray(np.repeat(Vp, G, axis=2).transpose(0, 2, 1, 3))
    inv = dtype(1.0 / math.sqrt(d))
    dQ = np.zeros((B, Hq, plan.Npad, d), dtype)
    dKx = np.zeros((B, Hq, plan.Lpad, d), dtype)
    dVx = np.zeros((B, Hq, plan.Lpad, d), dtype)
    bidx = np.arange(B)
    for i in (range(nq) if q_blocks is None else q_blocks):
        qs = slice(i * bs, (i + 1) * bs)
        q_idx = np.arange(i * bs, (i + 1) * bs)
        blocks = list(visited_key_blocks(i, nk, plan.window))
        kidx = np.concatenate([np.arange(j * bs, (j + 1) * bs) for j in blocks])
        Kb, Vb = Kh[:, :, kidx], Vh[:, :, kidx]
        # recompute the block's forward (all visited tiles at once)
        sc = np.exp(np.matmul(Qh[:, :, qs], Kb.transpose(0, 1, 3, 2)) * inv)
        sc *= _tile_mask(plan, bidx, q_idx, kidx)
        Z = sc.sum(axis=-1, keepdims=True)
        P = sc / np.where(Z > 0, Z, 1)
        g = dOh[:, :, qs]
        dP = np.matmul(g, Vb.transpose(0, 1, 3, 2))
        delta = (dP * P).sum(axis=-1, keepdims=True)
        dS = P * (dP - delta)
        dQ[:, :, qs] = np.matmul(dS, Kb) * inv
        dKx[:, :, kidx] += np.matmul(dS.transpose(0, 1, 3, 2), Qh[:, :, qs]) * inv
        dVx[:, :, kidx] += np.matmul(P.transpose(0, 1, 3, 2), g)
    dK = dKx.reshape(B, Hkv, G, plan.Lpad, d).sum(axis=2).transpose(0, 2, 1, 3)
    dV = dVx.reshape(B, Hkv, G, plan.Lpad, d).sum(axis=2).transpose(0, 2, 1, 3)
    return dQ.transpose(0, 2, 1, 3), dK, dV


def count_pairs(mask: np.ndarray) -> int:
    """Number of allowed (b, h, q, k) positions: the FLOP basis of the metric."""
    return int(np.count_nonzero(mask))
