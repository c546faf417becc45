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
  bfloat16 for dK and dQ, and dQ's dP from dO rounded to bfloat16.

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
    O = round_to(np.einsum("bhqk,bkhd->bqhd", Ph, Vx) / ls.transpose(0, 2, 1, 3), "float32")
    P = Pu / ls                                 # the backward's exp(S - lse)
    dOh = sig11(dO)
    Ot = np.transpose(O, (0, 2, 1, 3))
    delta = (np.transpose(dOh, (0, 2, 1, 3)) * Ot).sum(-1)[..., None]
    dP = np.einsum("bqhd,bkhd->bhqk", dOh, Vx)
    dS = P * (dP - delta)
    dVx = np.einsum("bhqk,bqhd->bkhd", sig11(P), dOh)
    if design == "float16":
        dSk = dSq = sig11(dS)
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
