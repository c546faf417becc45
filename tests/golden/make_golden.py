"""Writes the golden fixtures of this directory from the fp64 oracle.

Run from the repository root:  python tests/golden/make_golden.py

Each case stores its inputs exactly as the kernels receive them (float32, or
the raw 16-bit patterns of bfloat16 / float16 values), the upstream gradient
(bfloat16-representable values, stored as bits), the case description (JSON;
masks are named entries of MASKS in tests/golden/cases.py) and the oracle's
float64 results rounded to float32: O and the base-2 LSE, plus dQ, dK, dV
unless the case is forward-only.  The oracle itself is pinned by
tests/test_oracle.py; these files freeze its outputs so that a change to it,
or to the kernels, shows up as a difference against fixed data.
"""
import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

from oracle import attention_oracle as ao  # noqa: E402
from tests.golden.cases import CASES, encode, kwargs_of, round_to  # noqa: E402


def make_inputs(c):
    B, N, L, Hq, Hkv, d = c["shape"]
    gen = [np.random.Generator(np.random.PCG64(x)) for x in np.random.SeedSequence(c["seed"]).spawn(4)]
    f = d ** -0.25 if c.get("scaled", True) else 1.0
    Q = round_to(gen[0].standard_normal((B, N, Hq, d)) * f, c["dtype"])
    K = round_to(gen[1].standard_normal((B, L, Hkv, d)) * f, c["dtype"])
    V = round_to(gen[2].standard_normal((B, L, Hkv, d)) * f, c["dtype"])
    dO = round_to(gen[3].standard_normal((B, N, Hq, d)), "bfloat16")
    return Q, K, V, dO


def main():
    for name, c in CASES.items():
        Q, K, V, dO = make_inputs(c)
        plan = ao.canonical_plan(Q.shape, K.shape, V.shape, **kwargs_of(c))
        allowed = ao.effective_mask(plan)
        O, lse = ao.dense_forward(Q, K, V, allowed)
        out = dict(Q=encode(Q, c["dtype"]), K=encode(K, c["dtype"]), V=encode(V, c["dtype"]),
                   O=O.astype(np.float32), lse=lse.astype(np.float32), meta=json.dumps(c))
        if not c.get("forward_only"):
            dQ, dK, dV = ao.dense_backward(Q, K, V, allowed, dO)
            out.update(dO=encode(dO, "bfloat16"), dQ=dQ.astype(np.float32), dK=dK.astype(np.float32),
                       dV=dV.astype(np.float32))
        np.savez_compressed(os.path.join(HERE, f"{name}.npz"), **out)
        print(name, {k: v.shape for k, v in out.items() if k != "meta"})


if __name__ == "__main__":
    main()
