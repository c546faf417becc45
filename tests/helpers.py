"""Shared helpers of the parity tests: seeded inputs, the fp64 oracle wrapper,
and the tolerance checks the BASELINE parity gates define."""
from __future__ import annotations

import math

import numpy as np

from oracle import attention_oracle as ao

# Parity gate, element-wise, with b the fp64 oracle on the same rounded inputs:
#     |a - b| <= max(atol + rtol * |b|,  half_ulp(b) + SLACK * |b|)
# (atol, rtol) = (2e-3, 2e-3) for 16-bit inputs and (1e-5, 1e-5) for float32
# (the north star's tolerances).  The second term only matters where the
# first is below what the output dtype can represent: half_ulp(b) is the
# rounding of b to the OUTPUT dtype (zero for float32 outputs), and a
# bfloat16 value in [2, 2.9) is only known to 2^-7 > 2e-3 + 2e-3 |b|, so even
# the correctly rounded exact result fails the first term there
# (test_oracle_rounding_floor).  SLACK = 2^-10 is the error a result carries
# before that rounding from its 16-bit matrix-core operands: each product's
# two float16 operands (P, dS, dO are computed or float32 values) are rounded
# to half a float16 ulp, 2^-11 relative, each.  Where 2e-3 + 2e-3 |b| exceeds
# half an output ulp by more than that (|b| < ~1 for bfloat16 gradients),
# the first term alone decides.  The reference tests' norm-relative error is
# reported alongside.
SLACK = 2.0 ** -10
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


def oracle(Q, K, V, dO, kw, grads=True, scale=None):
    """fp64 closed-form O, base-2 LSE and gradients on exactly the given values.
    A ``kernel_fn`` in kw selects the softmax scale: the reference's
    threshold_kernel (attention.py:18-36) is exp(q.k - t / sqrt(d)), whose
    constant factor cancels in the normalisation -- scale 1; the default
    kernel's is 1/sqrt(d).  ``scale`` overrides both (a user kernel
    exp(s q.k + c) is a softmax with scale s)."""
    kw = dict(kw)
    kfn = kw.pop("kernel_fn", None)
    if scale is None:
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


def gate_bound(want, dtype_name, out_dtype_name=None):
    """Element-wise bound of the parity gate (see the top of this file)."""
    atol, rtol = TOL[dtype_name]
    want = np.abs(np.asarray(want, np.float64))
    g = atol + rtol * want
    h = half_ulp(want, out_dtype_name or dtype_name)
    return np.maximum(g, np.where(h > 0, h + SLACK * want, 0.0))


def assert_close(got, want, dtype_name, what="", out_dtype_name=None):
    """dtype_name picks (atol, rtol); out_dtype_name (default dtype_name) the
    output rounding term.  Prints and returns max(err / bound)."""
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    assert got.shape == want.shape, (what, got.shape, want.shape)
    assert np.all(np.isfinite(got)), f"{what}: non-finite values"
    err = np.abs(got - want)
    bound = gate_bound(want, dtype_name, out_dtype_name)
    ratio = float((err / bound).max()) if err.size else 0.0
    print(f"[gate] {what}: max err/bound {ratio:.3f}, norm-relative {norm_rel(got, want):.2e}")
    bad = err > bound
    if bad.any():
        i = np.unravel_index(np.argmax(err - bound), err.shape)
        raise AssertionError(
            f"{what}: {bad.sum()} of {bad.size} elements out of tolerance "
            f"(worst at {i}: got {got[i]:.6g}, want {want[i]:.6g}, |err| {err[i]:.3g}, "
            f"max err/bound {ratio:.3f}); norm-relative error {norm_rel(got, want):.3g}")
    return ratio


def assert_close_or_floor(got, want, dtype_name, what, floor, model, out_dtype_name=None):
    """assert_close, except for a known float16-operand floor: ``floor`` is the
    number of elements expected past the bound (0: none); each must also be
    past it in ``model(index)`` -- a float64 model of the kernels' roundings
    for that element, returning (value, sum of its terms' magnitudes) --
    rounded to the output dtype, and agree with the kernel's value to one
    output ulp plus the float32 accumulation error of up to 64 terms
    (64 * 2^-24 times the magnitudes).  A floor case that meets the gate fails
    too (the floor entry is then stale)."""
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    bound = gate_bound(want, dtype_name, out_dtype_name)
    err = np.abs(got - want)
    bad = np.argwhere(err > bound)
    if floor == 0 or len(bad) == 0:
        assert floor == 0, f"{what} now meets the gate: the float16-operand floor entry is stale"
        return assert_close(got, want, dtype_name, what, out_dtype_name)
    print(f"[gate] {what}: max err/bound {float((err / bound).max()):.3f} at {len(bad)} element(s) "
          f"(known float16-operand floor: {floor})")
    assert len(bad) == floor, (what, bad.tolist())
    out = out_dtype_name or dtype_name
    for idx in map(tuple, bad):
        m, mag = model(idx)
        mo = round_to_dtype(m, out)
        ulp = 2.0 * half_ulp(np.asarray([got[idx]]), out)[0] + 2.0 ** -18 * mag
        print(f"[floor] {what} at {idx}: kernel {got[idx]:.6g}, operand-rounding model {m:.6g} -> "
              f"{mo:.6g}, exact {want[idx]:.6g}, bound {bound[idx]:.3g}", flush=True)
        assert abs(mo - want[idx]) > bound[idx], "the rounding model meets the gate here: not the floor"
        assert abs(mo - got[idx]) <= ulp, "the kernel differs from the rounding model"


def round_to_dtype(x, name):
    """x (a float) rounded to the named dtype, as a float."""
    import torch

    return float(torch.tensor(float(x), dtype=torch.float64).to(getattr(torch, name)).double())


def norm_rel(a, b):
    """The reference tests' metric, ||a - b|| / min(||a||, ||b||) (test_mapped_attention.py:275-300)."""
    na, nb = np.linalg.norm(a), np.linalg.norm(b)
    den = min(na, nb)
    return float(np.linalg.norm(a - b) / den) if den > 0 else float(np.linalg.norm(a - b))
