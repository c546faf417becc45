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


def _draw(seed):
    from tests.test_random_sweep_gpu import draw

    c = draw(seed)
    B, N, L, Hq, Hkv, d = c["shape"]
    Q, K, V, dO = seeded_inputs(B, N, L, Hq, Hkv, d, seed)
    scale = 1.0 if "kernel_fn" in c["kw"] else 1 / math.sqrt(d)
    assert c["dtype"] == "bfloat16"
    return Q, K, V, dO, c["kw"], scale, c["out"] or "float32"


@pytest.mark.parametrize("seed", [25, 100, 165])
def test_float16_operands_fix_known_draws(seed):
    Q, K, V, dO, kw, scale, out = _draw(seed)
    assert max(_ratios(Q, K, V, dO, kw, "bfloat16", scale, "bfloat16", out)) > 1.5
    assert max(_ratios(Q, K, V, dO, kw, "bfloat16", scale, "float16", out)) <= 1.0


# (draw, gradient index 0 dQ / 1 dK / 2 dV, the ratio the GPU reports)
FLOOR = [(31, 1, 1.007), (94, 2, 1.004), (118, 1, 1.514),
         (647, 0, 1.015), (696, 2, 1.051), (976, 2, 1.024)]


@pytest.mark.parametrize("seed,which,gpu", FLOOR)
def test_float16_floor_draws(seed, which, gpu):
    Q, K, V, dO, kw, scale, out = _draw(seed)
    r = _ratios(Q, K, V, dO, kw, "bfloat16", scale, "float16", out)
    assert r[which] == pytest.approx(gpu, abs=0.02), r


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
