"""Shared helpers of the parity tests: seeded inputs, the fp64 oracle wrapper,
and the tolerance checks the BASELINE parity gates define."""
from __future__ import annotations

import math

import numpy as np

from oracle import attention_oracle as ao

# Parity gate, element-wise:
#     |a - b| <= atol + rtol * |b| + half_ulp(b)
# with (atol, rtol) = (2e-3, 2e-3) for 16-bit inputs and (1e-5, 1e-5) for
# float32 (the north star's tolerances), b the fp64 oracle on the same rounded
# inputs, and half_ulp(b) the rounding of b to the OUTPUT dtype (zero for a
# float32 output).  The last term is what even the correctly rounded exact
# result incurs: a bfloat16 value in [2, 4) is only known to 2^-7, more than
# 2e-3 + 2e-3 * |b| (test_oracle_rounding_floor shows the bare gate fails for
# bf16(exact)).  The reference tests' norm-relative error is reported alongside.
TOL = {"bfloat16": (2e-3, 2e-3), "float16": (2e-3, 2e-3), "float32": (1e-5, 1e-5)}
_SIG = {"bfloat16": (8, -126), "float16": (11, -14)}   # significand bits, min normal exponent


def half_ulp(b, out_dtype_name):
    """Half a unit in the last place of b in the output dtype (0 for float32)."""
    if out_dtype_name not in _SIG:
        return np.zeros_like(np.asarray(b, np.float64))
    p, emin = _SIG[out_dtype_name]
    b = np.abs(np.asarray(b, np.float64))
    e = np.floor(np.log2(np.where(b > 0, b, 1.0)))
    e = np.where(b > 0, np.maximum(e, emin), emin)
    return 2.0 ** (e - p)


def seeded_inputs(B, N, L, Hq, Hkv, d, seed, scaled=True):
    """Q, K, V, dO as float32 numpy arrays, N(0,1) (times d^-0.25 when scaled),
    from independent PCG64 streams."""
    ss = np.random.SeedSequence(seed).spawn(4)
    f = d ** -0.25 if scaled else 1.0
    Q = np.random.Generator(np.random.PCG64(ss[0])).standard_normal((B, N, Hq, d)).astype(np.float32) * f
    K = np.random.Generator(np.random.PCG64(ss[1])).standard_normal((B, L, Hkv, d)).astype(np.float32) * f
    V = np.random.Generator(np.random.PCG64(ss[2])).standard_normal((B, L, Hkv, d)).astype(np.float32) * f
    dO = np.random.Generator(np.random.PCG64(ss[3])).standard_normal((B, N, Hq, d)).astype(np.float32)
    return Q, K, V, dO


def oracle(Q, K, V, dO, kw, grads=True):
    """fp64 closed-form O, base-2 LSE and gradients on exactly the given values.
    A ``kernel_fn`` in kw selects the softmax scale: the reference's
    threshold_kernel (attention.py:18-36) is exp(q.k - t / sqrt(d)), whose
    constant factor cancels in the normalisation -- scale 1; the default
    kernel's is 1/sqrt(d)."""
    kw = dict(kw)
    kfn = kw.pop("kernel_fn", None)
    scale = None if kfn is None or getattr(kfn, "_mattn_scale", None) is None else float(kfn._mattn_scale)
    plan = ao.canonical_plan(Q.shape, K.shape, V.shape, **kw)
    Qb, Kb, Vb, dOb = (x if x is None or not plan.squeeze_batch else x[None] for x in (Q, K, V, dO))
    allowed = ao.effective_mask(plan)
    O, lse = ao.dense_forward(Qb, Kb, Vb, allowed, scale=scale)
    g = ao.dense_backward(Qb, Kb, Vb, allowed, dOb, scale=scale) if grads else None
    if plan.squeeze_batch:
        O = O[0]
        g = tuple(x[0] for x in g) if g is not None else None
    return O, lse / math.log(2.0), g, allowed


def assert_close(got, want, dtype_name, what="", out_dtype_name=None):
    """dtype_name picks (atol, rtol); out_dtype_name (default dtype_name) the
    output rounding term."""
    atol, rtol = TOL[dtype_name]
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    assert got.shape == want.shape, (what, got.shape, want.shape)
    assert np.all(np.isfinite(got)), f"{what}: non-finite values"
    err = np.abs(got - want)
    bound = atol + rtol * np.abs(want) + half_ulp(want, out_dtype_name or dtype_name)
    bad = err > bound
    if bad.any():
        i = np.unravel_index(np.argmax(err - bound), err.shape)
        raise AssertionError(
            f"{what}: {bad.sum()} of {bad.size} elements out of tolerance "
            f"(worst at {i}: got {got[i]:.6g}, want {want[i]:.6g}, |err| {err[i]:.3g}); "
            f"norm-relative error {norm_rel(got, want):.3g}")


def norm_rel(a, b):
    """The reference tests' metric, ||a - b|| / min(||a||, ||b||) (test_mapped_attention.py:275-300)."""
    na, nb = np.linalg.norm(a), np.linalg.norm(b)
    den = min(na, nb)
    return float(np.linalg.norm(a - b) / den) if den > 0 else float(np.linalg.norm(a - b))
