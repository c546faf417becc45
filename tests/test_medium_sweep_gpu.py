"""Seeded random problems of medium size against the fp64 oracle: lengths
drawn from 500-2500 (several 128-row tiles per column and row, ragged ends),
GQA, D 64 or 128, bfloat16 or float16, block size 64 or 128, and one mask
family per draw: causal, causal sliding window, packed documents, no mask,
per-head tile table.  The committed draws cover lengths 649-1548 and up to
eight (b, head) groups: seeds 0-4, and seed 12 of a one-off 40-problem run,
whose float16 document problem left one dV element 0.2% past the gate with
the kernels' earlier operands.  Same gate as the small sweep (tests/helpers.py)."""
import numpy as np
import pytest

from tests.helpers import Floor, assert_close, oracle, seeded_inputs

torch = pytest.importorskip("torch")

pytestmark = pytest.mark.gpu

FAMILIES = ["causal", "window", "docs", "none", "table"]


def draw(seed):
    from jaxmodules_amd import masks

    rng = np.random.default_rng(5000 + seed)
    B = int(rng.integers(1, 3))
    Hkv = int(rng.choice([1, 2, 4, 8]))
    Hq = Hkv * int(rng.choice([1, 2]))
    d = int(rng.choice([64, 128]))
    dtype = str(rng.choice(["bfloat16", "float16"]))
    bs = int(rng.choice([64, 128]))
    N = int(rng.integers(500, 2500))
    fam = FAMILIES[seed % len(FAMILIES)]
    kw = dict(block_size=bs)
    if fam == "causal":
        kw["is_causal"] = True
    elif fam == "window":
        left = int(rng.integers(50, 800))
        kw["mask_fn"] = masks.intersect(masks.window(left, 0), masks.causal())
    elif fam == "docs":
        lens = rng.integers(20, 600, size=64)
        doc = np.repeat(np.arange(64), lens)[:N]
        doc = np.concatenate([doc, np.full(max(0, N - len(doc)), 64)])
        kw["mask_fn"] = masks.intersect(masks.documents(doc), masks.causal())
    elif fam == "table":
        nt = -(-N // 128)
        tbl = (rng.random((Hq, nt, nt)) < 0.4).astype(np.uint8) * 2
        kw["mask_fn"] = masks.intersect(masks.tile_table(tbl), masks.causal())
    return dict(shape=(B, N, N, Hq, Hkv, d), kw=kw, dtype=dtype, fam=fam)


def run_medium(seed, precision=None):
    """One draw against the oracle; a default-path miss within the float16
    operands' bound (tests/helpers.py Floor) reruns it at precision
    "highest", which must meet the gate, and then xfails."""
    import jaxmodules_amd as jm

    c = draw(seed)
    B, N, L, Hq, Hkv, d = c["shape"]
    print(f"[medium] seed={seed} {c['fam']} shape={c['shape']} dtype={c['dtype']} "
          f"block={c['kw']['block_size']} precision={precision}", flush=True)
    Q, K, V, dO = seeded_inputs(B, N, L, Hq, Hkv, d, 9000 + seed)
    td = getattr(torch, c["dtype"])
    q, k, v = (torch.from_numpy(x).to("cuda", td).requires_grad_() for x in (Q, K, V))
    o = jm.masked_attention_via_map(q, k, v, precision=precision, **c["kw"])
    Qr, Kr, Vr = (x.detach().float().cpu().numpy() for x in (q, k, v))
    do_t = torch.from_numpy(dO).to("cuda", o.dtype)
    O_ref, _, g_ref, _ = oracle(Qr, Kr, Vr, do_t.float().cpu().numpy(), c["kw"])
    floor = Floor() if precision is None else None
    assert_close(o.detach().float().cpu().numpy(), O_ref, c["dtype"], "O", str(o.dtype).replace("torch.", ""),
                 floor=floor)
    o.backward(do_t)
    for name, t, r in (("dQ", q, g_ref[0]), ("dK", k, g_ref[1]), ("dV", v, g_ref[2])):
        assert_close(t.grad.float().cpu().numpy(), r, c["dtype"], name, floor=floor)
    torch.cuda.synchronize()
    if floor is not None and floor.misses:
        run_medium(seed, precision="highest")
        floor.finish()


@pytest.mark.parametrize("seed", [0, 1, 2, 3, 4, 12])
def test_medium_problem(seed):
    run_medium(seed)


def test_draws_cover_every_family():
    assert {draw(s)["fam"] for s in range(5)} == set(FAMILIES)
