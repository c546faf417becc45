"""The parity-gate misses of the 16-bit path, explained on the CPU with the
model of the kernels' roundings (tests/rounding_model.py) against the fp64
oracle, under the same gate as the GPU tests (tests/helpers.py):

* the known draws of the 600-problem sweep exceed the gate with bfloat16 dS
  and dO operands (the earlier kernels) and pass with float16 ones;
* the draws that still miss with float16 operands (strict xfails in
  tests/test_random_sweep_gpu.py and tests/test_regimes_gpu.py) miss in the
  model too, by the same ratio the GPU reports -- single elements whose sums
  of rounded products cancel: the floor of 16-bit operands.
"""
import math

import numpy as np
import pytest

from tests.helpers import gate_bound, oracle, seeded_inputs
from tests.rounding_model import kernel_model, round_to


def _ratios(Q, K, V, dO, kw, dtype, scale, design, out="float32"):
    """max(err / bound) of dQ, dK, dV; dO arrives in the output dtype ``out``."""
    Qr, Kr, Vr = (round_to(x, dtype) for x in (Q, K, V))
    dOr = round_to(dO, out)
    O_ref, _, g_ref, allowed = oracle(Qr, Kr, Vr, dOr, kw)
    out = kernel_model(Qr, Kr, Vr, dOr, allowed, scale, dtype, design)
    return [float((np.abs(a - b) / gate_bound(b, dtype, dtype)).max()) for a, b in zip(out[1:], g_ref)]


def _draw(seed, dtype="bfloat16"):
    from tests.test_random_sweep_gpu import draw

    c = draw(seed)
    B, N, L, Hq, Hkv, d = c["shape"]
    Q, K, V, dO = seeded_inputs(B, N, L, Hq, Hkv, d, seed)
    scale = 1.0 if "kernel_fn" in c["kw"] else 1 / math.sqrt(d)
    assert c["dtype"] == dtype
    return Q, K, V, dO, c["kw"], scale, c["out"] or "float32"


@pytest.mark.parametrize("seed", [25, 100, 165])
def test_float16_operands_fix_known_draws(seed):
    Q, K, V, dO, kw, scale, out = _draw(seed)
    assert max(_ratios(Q, K, V, dO, kw, "bfloat16", scale, "bfloat16", out)) > 1.5
    assert max(_ratios(Q, K, V, dO, kw, "bfloat16", scale, "float16", out)) <= 1.0


# (draw, gradient index 0 dQ / 1 dK / 2 dV, the ratio the GPU reports[, dtype])
FLOOR = [(31, 1, 1.007), (94, 2, 1.004), (118, 1, 1.514),
         (647, 0, 1.015), (696, 2, 1.051), (976, 2, 1.024),
         (1060, 2, 1.026), (1067, 2, 1.052), (1073, 2, 1.035), (1193, 2, 1.002), (1201, 2, 1.013),
         (1246, 2, 1.049), (1271, 2, 1.302, "float16"), (1288, 2, 1.113), (1414, 2, 1.026)]


@pytest.mark.parametrize("case", FLOOR, ids=[str(c[0]) for c in FLOOR])
def test_float16_floor_draws(case):
    seed, which, gpu = case[:3]
    dtype = case[3] if len(case) > 3 else "bfloat16"
    Q, K, V, dO, kw, scale, out = _draw(seed, dtype)
    r = _ratios(Q, K, V, dO, kw, dtype, scale, "float16", out)
    assert r[which] == pytest.approx(gpu, abs=0.02), r


def test_float16_floor_draw_at_a_rounding_midpoint():
    """Draw 1120: the GPU returns dV[2, 1, 0, 35] one bfloat16 ulp above the
    exact 1.2213751 (1.017x the bound), the model one below.  The model's
    unrounded sum of float16-rounded products lies within 2e-6 of the
    midpoint 1.22265625 between the two, 0.00128 above the exact value: the
    float16 floor again, with the last float32 bits (summation order, the
    forward's lse) deciding the rounding."""
    from tests.rounding_model import _expand, f16, round_to, sig11

    Q, K, V, dO, kw, scale, out = _draw(1120)
    Qr, Kr = round_to(Q, "bfloat16"), round_to(K, "bfloat16")
    dOr = round_to(dO, out)
    _, _, g_ref, allowed = oracle(Qr, Kr, round_to(V, "bfloat16"), dOr, kw)
    Hq = Q.shape[2]
    S = np.where(allowed, np.einsum("bqhd,bkhd->bhqk", Qr, _expand(Kr, Hq)) * scale, -np.inf)
    m = S.max(-1, keepdims=True)
    Pu = np.where(allowed, np.exp(S - np.where(np.isfinite(m), m, 0.0)), 0.0)
    l = f16(Pu).sum(-1, keepdims=True)
    P = Pu / np.where(l > 0, l, 1.0)
    b, k, hk, col = 2, 1, 0, 35
    G = Hq // K.shape[2]
    v = sum(float((sig11(P[b, h, :, k]) * sig11(dOr)[b, :, h, col]).sum()) for h in range(hk * G, hk * G + G))
    assert abs(v - 1.22265625) < 2e-6
    assert v - g_ref[2][b, k, hk, col] == pytest.approx(0.00128, abs=1e-5)


def test_float16_floor_unit_normal_causal():
    from tests.test_regimes_gpu import _mask_kw

    B, N, Hq, Hkv, d = 2, 300, 4, 2, 64
    Q, K, V, dO = seeded_inputs(B, N, N, Hq, Hkv, d, 4242 + N + d, scaled=False)
    kw = _mask_kw("causal", N, 64)
    assert max(_ratios(Q, K, V, dO, kw, "bfloat16", 1 / 8, "bfloat16")) > 2
    r = _ratios(Q, K, V, dO, kw, "bfloat16", 1 / 8, "float16")
    assert r[0] < 1 and r[1] < 1 and r[2] == pytest.approx(1.10, abs=0.02), r


def test_residue_dv_model_without_roundings_is_exact(monkeypatch):
    """residue_dv_model with the roundings switched off equals dV of the dense
    float64 attention under the strided causal mask (k % P == q % P, k <= q)."""
    import math

    from tests import rounding_model as rm

    rng = np.random.default_rng(0)
    L, d, P = 600, 16, 64
    Q, K, dO = rng.standard_normal((L, d)), rng.standard_normal((L, d)), rng.standard_normal((L, d))
    q, k = np.arange(L)[:, None], np.arange(L)[None, :]
    allowed = (k <= q) & ((q - k) % P == 0)
    s = np.where(allowed, Q @ K.T / math.sqrt(d), -np.inf)
    p = np.exp(s - s.max(1, keepdims=True))
    p /= p.sum(1, keepdims=True)
    dV = p.T @ dO
    monkeypatch.setattr(rm, "sig11", lambda x: np.asarray(x, np.float64))
    for key, col in [(0, 3), (70, 5), (599, 0), (64, 15)]:
        assert math.isclose(rm.residue_dv_model(Q, K, dO, P, key, col, 1 / math.sqrt(d))[0], dV[key, col],
                            rel_tol=1e-12, abs_tol=1e-14)
