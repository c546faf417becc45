"""Golden fixtures (tests/golden/*.npz, written by tests/golden/make_golden.py).

CPU: the oracle, re-run on the stored inputs, reproduces the stored outputs
(to float32 storage precision), and the host tracer's tile map expands to the
mask the fixture was computed under.
GPU: the HIP path, through the C ABI, against the stored outputs under the
parity gate (2e-3 + 2e-3 |b| for 16-bit inputs, 1e-5 for float32, plus half an
ulp of the output dtype); the base-2 LSE the forward kernel writes against the
stored natural-log LSE.
"""
import glob
import json
import math
import os

import numpy as np
import pytest

from oracle import attention_oracle as ao
from tests.golden.cases import CASES, decode, kwargs_of
from tests.helpers import Floor, assert_close, magnitudes

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
NAMES = sorted(os.path.basename(p)[:-4] for p in glob.glob(os.path.join(HERE, "*.npz")))


def load(name):
    with np.load(os.path.join(HERE, name + ".npz")) as z:
        f = {k: z[k] for k in z.files}
    c = json.loads(str(f.pop("meta")))
    dt = c["dtype"]
    for k in ("Q", "K", "V"):
        f[k] = decode(f[k], dt)
    if "dO" in f:
        f["dO"] = decode(f["dO"], "bfloat16")
    return c, f


def test_every_case_has_a_fixture():
    assert sorted(CASES) == NAMES


@pytest.mark.parametrize("name", NAMES)
def test_oracle_reproduces_fixture(name):
    c, f = load(name)
    assert c == json.loads(json.dumps(CASES[name]))  # the case list and the fixture agree
    plan = ao.canonical_plan(f["Q"].shape, f["K"].shape, f["V"].shape, **kwargs_of(c))
    allowed = ao.effective_mask(plan)
    O, lse = ao.dense_forward(f["Q"], f["K"], f["V"], allowed)
    np.testing.assert_allclose(O, f["O"], rtol=1e-6, atol=1e-7)
    fin = np.isfinite(f["lse"])
    assert np.array_equal(fin, np.isfinite(lse))
    np.testing.assert_allclose(lse[fin], f["lse"][fin], rtol=1e-6, atol=1e-7)
    if "dQ" in f:
        for got, k in zip(ao.dense_backward(f["Q"], f["K"], f["V"], allowed, f["dO"]), ("dQ", "dK", "dV")):
            np.testing.assert_allclose(got, f[k], rtol=1e-6, atol=1e-7)


@pytest.mark.parametrize("name", NAMES)
def test_tracer_mask_matches_fixture_case(name):
    from jaxmodules_amd import blockmap as bm

    c, f = load(name)
    kw = kwargs_of(c)
    ref = ao.effective_mask(ao.canonical_plan(f["Q"].shape, f["K"].shape, f["V"].shape, **kw))
    tm = bm.trace(bm.make_plan(f["Q"].shape, f["K"].shape, f["V"].shape, **kw))
    assert np.array_equal(np.broadcast_to(tm.dense(), ref.shape), ref)
    # the stored LSE is -inf exactly on the rows the mask leaves empty
    assert np.array_equal(~np.isfinite(f["lse"]), ~ref.any(axis=-1))


@pytest.mark.gpu
@pytest.mark.parametrize("name", NAMES)
def test_hip_path_matches_fixture(name):
    torch = pytest.importorskip("torch")
    import jaxmodules_amd as jm
    from jaxmodules_amd import attention as at

    print(f"[golden] {name}", flush=True)
    c, f = load(name)
    dt = c["dtype"]
    td = getattr(torch, dt)
    kw = kwargs_of(c)
    grads = "dQ" in f
    q, k, v = (torch.from_numpy(f[x]).to("cuda", td).requires_grad_(grads) for x in ("Q", "K", "V"))
    o = jm.masked_attention_via_map(q, k, v, **kw)
    # the terms' magnitudes of the gate's accumulation slack, from the fixture's inputs
    Qr, Kr, Vr = (x.detach().double().cpu().numpy() for x in (q, k, v))
    plan = ao.canonical_plan(Qr.shape, Kr.shape, Vr.shape, **kw)
    sq = (lambda x: x[None]) if plan.squeeze_batch else (lambda x: x)
    un = (lambda x: x[0]) if plan.squeeze_batch else (lambda x: x)
    mags = [None if m is None else un(m) for m in magnitudes(
        sq(Qr), sq(Kr), sq(Vr), ao.effective_mask(plan), sq(f["dO"].astype(np.float64)) if grads else None)]
    floor = Floor() if dt != "float32" else None
    assert_close(o.detach().float().cpu().numpy(), f["O"], dt, f"{name} O", "float32", mag=mags[0], floor=floor)

    plan, tm = at.trace_call(tuple(q.shape), tuple(k.shape), tuple(v.shape), **kw)
    _, lse2, _ = at.mattn_forward(q.detach(), k.detach(), v.detach(), tm, 1.0 / math.sqrt(c["shape"][-1]))
    lse = lse2.cpu().numpy().astype(np.float64) * math.log(2.0)
    fin = np.isfinite(f["lse"])
    assert np.array_equal(np.isfinite(lse), fin)
    assert_close(lse[fin], f["lse"][fin], dt, f"{name} LSE", "float32")

    if grads:
        o.backward(torch.from_numpy(f["dO"]).to("cuda"))
        for (x, t), m in zip((("dQ", q), ("dK", k), ("dV", v)), mags[1:]):
            assert t.grad.dtype == td
            assert_close(t.grad.float().cpu().numpy(), f[x], dt, f"{name} {x}", mag=m, floor=floor)
    torch.cuda.synchronize()
    if floor is not None:
        floor.finish()
