"""A float64 model of the 16-bit kernels' roundings (test infrastructure).

It computes what the HIP path computes, with every operand rounded exactly
where the kernels round it and float64 arithmetic everywhere else (the
kernels accumulate in float32; that difference is far below the operand
roundings).  Two designs are modelled:

* ``"float16"`` -- the kernels of this repository: the forward multiplies P
  rounded to float16 with V (exact in float16 after a power-of-two scale) and
  sums the rounded P for the row normaliser; the backward rounds P, dS and dO
  to float16 (Q, K, V exact after their scales) and takes delta from the
  float32 O and the float16 dO;
* ``"bfloat16"`` -- the earlier operand choice for bfloat16 inputs: P in the
  input dtype for P V with the normaliser from the unrounded P, dS in
  bfloat16 for dK and dQ, and dQ's dP from dO rounded to bfloat16;
* ``"split"`` -- the float16 design with split rows, as the kernels run it
  now: a row that puts a weight of at least SPLIT_P on a key has its O and
  lse formed again from unrounded weights and their sum, and enters the
  backward with its float16 operands' rounded-off parts (dO, P and dS to 22
  significant bits, i.e. unrounded here) and delta from the unrounded dO;
  the other rows as ``"float16"`` (the kernels also take the rounded-off parts
  of those rows' terms where they share a sub-block with a split row's
  allowed pairs; the model leaves them rounded, the weaker case).

Operands the kernels scale by a power of two before rounding (dO, the
backward's P and dS) are rounded to float16's 11 significant bits without its
exponent limits (sig11); the forward's unscaled P is rounded to float16
itself.  Used by tests/test_rounding_model.py to show which parity-gate
misses are the floor of 16-bit operands.
"""
from __future__ import annotations

import numpy as np
import torch


def bf16(x):
    return torch.from_numpy(np.asarray(x, np.float32)).to(torch.bfloat16).double().numpy()


def f16(x):
    return np.asarray(x, np.float32).astype(np.float16).astype(np.float64)


def sig11(x):
    """x rounded to 11 significant bits (float16's), any exponent: float16
    rounding of x times a power of two that puts it in float16's normal range."""
    x = np.asarray(x, np.float32).astype(np.float64)
    mant, e = np.frexp(x)                      # x = mant 2^e, |mant| in [0.5, 1)
    return np.ldexp(np.round(mant * 2048.0) / 2048.0, e)   # round-half-even on the 11 bits


def round_to(x, name):
    if name == "bfloat16":
        return bf16(x)
    if name == "float16":
        return f16(x)
    return np.asarray(x, np.float32).astype(np.float64)


def _expand(X, Hq):
    return np.repeat(X, Hq // X.shape[2], axis=2)


SPLIT_P = 1 / 32  # largest weight from which a query tile is split (common.hpp SPLIT_P)
TILE = 128


def split_rows(P):
    """[B, Hq, N] booleans: the split rows, whose largest weight reaches SPLIT_P
    (P: [B, Hq, N, L] weights)."""
    return P.max(-1) >= SPLIT_P


def split_tiles(P):
    """[B, Hq, N] booleans: the rows of the 128-row query tiles holding a split row."""
    B, Hq, N, _ = P.shape
    nt = -(-N // TILE)
    pad = np.zeros((B, Hq, nt * TILE), bool)
    pad[..., :N] = split_rows(P)
    return np.repeat(pad.reshape(B, Hq, nt, TILE).any(-1), TILE, axis=-1)[..., :N]


def kernel_model(Q, K, V, dO, allowed, scale, dtype, design="float16"):
    """(O float32, dQ, dK, dV in dtype) for inputs already rounded to dtype and
    dO in float32; allowed is the [B, Hq, N, L] effective mask."""
    B, N, Hq, d = Q.shape
    Hkv, L = K.shape[2], K.shape[1]
    G = Hq // Hkv
    Kx, Vx = _expand(K, Hq), _expand(V, Hq)
    S = np.einsum("bqhd,bkhd->bhqk", Q, Kx) * scale
    S = np.where(allowed, S, -np.inf)
    m = S.max(-1, keepdims=True)
    m = np.where(np.isfinite(m), m, 0.0)
    Pu = np.where(allowed, np.exp(S - m), 0.0)
    if design == "float16":
        Ph = f16(Pu)
        l = Ph.sum(-1, keepdims=True)          # the normaliser of the rounded weights
    else:
        Ph = round_to(Pu, dtype)
        l = Pu.sum(-1, keepdims=True)
    ls = np.where(l > 0, l, 1.0)
    split = split_rows(Pu / ls) if design == "split" else np.zeros(Pu.shape[:3], bool)
    sq = split[..., None]                       # [B, Hq, N, 1]
    if design == "split":  # split rows: the forward again with unrounded weights and their sum
        Ph = np.where(sq, Pu, Ph)
        ls = np.where(sq, Pu.sum(-1, keepdims=True), ls)
        ls = np.where(ls > 0, ls, 1.0)
    O = round_to(np.einsum("bhqk,bkhd->bqhd", Ph, Vx) / ls.transpose(0, 2, 1, 3), "float32")
    P = Pu / ls                                 # the backward's exp(S - lse)
    dOh = np.where(np.transpose(split, (0, 2, 1))[..., None], np.asarray(dO, np.float64), sig11(dO))
    Ot = np.transpose(O, (0, 2, 1, 3))
    delta = (np.transpose(dOh, (0, 2, 1, 3)) * Ot).sum(-1)[..., None]
    dP = np.einsum("bqhd,bkhd->bhqk", dOh, Vx)
    dS = P * (dP - delta)
    dVx = np.einsum("bhqk,bqhd->bkhd", np.where(sq, P, sig11(P)), dOh)
    if design in ("float16", "split"):
        dSk = dSq = np.where(sq, dS, sig11(dS))
    else:
        dSk = bf16(dS)
        dO16 = bf16(dO)
        delta16 = (np.transpose(dO16, (0, 2, 1, 3)) * Ot).sum(-1)[..., None]
        dSq = bf16(P * (np.einsum("bqhd,bkhd->bhqk", dO16, Vx) - delta16))
    dKx = np.einsum("bhqk,bqhd->bkhd", dSk, Q) * scale
    dQ = np.einsum("bhqk,bkhd->bqhd", dSq, Kx) * scale
    dK = dKx.reshape(B, L, Hkv, G, d).sum(3)
    dV = dVx.reshape(B, L, Hkv, G, d).sum(3)
    return O, round_to(dQ, dtype), round_to(dK, dtype), round_to(dV, dtype)


# log2(1 + 2^-11): how far a sum of float16-rounded positive terms moves log2 of the sum
LSE_ROUNDING = float(np.log2(1.0 + 2.0 ** -11))


def residue_dv_model(Q, K, dO, period, key, col, scale, lse2=None):
    """dV[key, col] of one head under the strided causal mask k % P == q % P,
    k <= q (check_attn.py:9-32), as the float16 design rounds it: the sum over
    the queries of the key's residue class of sig11(P) sig11(dO).  P is
    exp2(s log2(e) - lse2[q]) with ``lse2`` the forward's base-2 log-sum-exp
    per row -- the log of the sum of the forward's float16-rounded weights
    (the self-consistent normaliser), checked here to lie within LSE_ROUNDING
    of the exact one -- or the exact softmax when ``lse2`` is None.
    Q, K: [L, d], dO: [L, d] (float64-exact copies of the kernel's inputs).
    Returns (value, sum of the terms' magnitudes)."""
    L = Q.shape[0]
    total, mag = 0.0, 0.0
    for q in range(key, L, period):
        ks = np.arange(q % period, q + 1, period)
        s = (K[ks] @ Q[q]) * scale
        m = s.max()
        exact2 = float((m + np.log(np.exp(s - m).sum())) / np.log(2.0))
        if lse2 is None:
            p = np.exp(s - m) / np.exp(s - m).sum()
        else:
            assert abs(float(lse2[q]) - exact2) <= LSE_ROUNDING + 1e-6, (q, float(lse2[q]), exact2)
            p = np.exp2(s / np.log(2.0) - float(lse2[q]))
        t = float(sig11(p[ks == key])[0] * sig11(dO[q, col]))
        total += t
        mag += abs(t)
    return total, mag
