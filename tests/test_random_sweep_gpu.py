"""A seeded random sweep of problem shapes and masks: the HIP path against the
fp64 oracle under the parity gate of tests/helpers.py.  Each case draws batch
size, query/key lengths (1..400, often ragged), GQA layout, head dim
(16..128, padded to 64/128 by the host), dtype, block size, kernel function,
output dtype and one mask family: causal, none, an element window with the
reference's block window, packed documents, a per-head tile table, a
head-specific lambda, or cross lengths.  The draw is fixed by the seed, so
every run checks the same problems: seeds 0-23, the draws of a one-off
600-problem run (seeds 24-623) that failed the gate with the kernels' earlier
bfloat16 dS / dO operands (KNOWN_DRAWS), the draws of two more one-off runs
(seeds 624-1423) that missed it with float16 operands (LATER_DRAWS), and the
draw of an 800-problem run (seeds 1424-2223) that missed it with split tiles
at their first threshold (SPLIT_DRAWS), and the draw of another (seeds
2224-3023) that misses it within the float16 operands' bound (FLOOR_DRAWS).

threshold_kernel is a softmax with scale 1 instead of 1/sqrt(d), so its
draws see logits of unit variance (Q, K ~ N(0,1) d^-0.25), seven times
sharper than the default kernel's at d = 48; precision None selects float32
arithmetic for them ("highest", attention.use_precise).  A default-path draw
that misses the gate only within the float16 operands' error bound
(tests/helpers.py Floor) is run again at precision "highest", which must meet
the gate, and is then reported xfailed."""
import numpy as np
import pytest

from tests.helpers import Floor, assert_close, oracle, seeded_inputs

torch = pytest.importorskip("torch")

pytestmark = pytest.mark.gpu

FAMILIES = ["causal", "none", "window", "docs", "table", "head", "cross"]


def draw(seed):
    from jaxmodules_amd import attention as A
    from jaxmodules_amd import masks

    rng = np.random.default_rng(1000 + seed)
    fam = FAMILIES[seed % len(FAMILIES)]
    B = int(rng.integers(1, 4))
    Hkv = int(rng.choice([1, 2, 4]))
    Hq = Hkv * int(rng.choice([1, 2]))
    d = int(rng.choice([16, 32, 48, 64, 80, 96, 128]))
    dtype = str(rng.choice(["bfloat16", "float16"]))
    bs = int(rng.choice([16, 32, 64, 128]))
    N = int(rng.integers(1, 401))
    L = N if fam != "cross" else int(rng.integers(1, 401))
    kw = dict(block_size=bs)
    if rng.random() < 0.3:
        kw["kernel_fn"] = A.threshold_kernel(float(rng.normal()))
    if fam == "causal":
        kw["is_causal"] = True
    elif fam == "window":
        left, right = int(rng.integers(0, 200)), int(rng.integers(0, 40))
        nk = -(-(L + (bs - L % bs if N % bs else 0)) // bs)
        lwb, rwb = -(-left // bs), 1 + -(-right // bs)
        if lwb + rwb <= nk:
            kw["window_size"] = (left, right)
        kw["mask_fn"] = masks.intersect(masks.window(left, right), masks.causal()) \
            if rng.random() < 0.5 else masks.window(left, right)
    elif fam == "docs":
        lens = rng.integers(1, 80, size=64)
        doc = np.repeat(np.arange(64), lens)[:N]
        doc = np.concatenate([doc, np.full(max(0, N - len(doc)), 64)])
        kw["mask_fn"] = masks.intersect(masks.documents(doc), masks.causal())
    elif fam == "table":
        nt_q, nt_k = -(-N // 128), -(-L // 128)
        tbl = rng.integers(0, 3, size=(Hq, nt_q, nt_k)).astype(np.uint8)
        kw["mask_fn"] = masks.intersect(masks.tile_table(tbl), masks.causal())
    elif fam == "head":
        kw["mask_fn"] = lambda b, h, q, k: ((q + h) % 3 != 0) & (k <= q + 2 * b)
    elif fam == "cross":
        kw["mask_fn"] = lambda b, h, q, k: (k * 2 <= q * 3 + 5)
    out = None if rng.random() < 0.7 else dtype
    return dict(shape=(B, N, L, Hq, Hkv, d), kw=kw, dtype=dtype, out=out, fam=fam)


def run_draw(seed, precision=None):
    import jaxmodules_amd as jm
    from jaxmodules_amd import attention as A

    c = draw(seed)
    B, N, L, Hq, Hkv, d = c["shape"]
    print(f"[sweep] seed={seed} {c['fam']} shape={c['shape']} dtype={c['dtype']} out={c['out']} "
          f"precision={precision} kw={ {k: v for k, v in c['kw'].items() if k != 'mask_fn'} }", flush=True)
    Q, K, V, dO = seeded_inputs(B, N, L, Hq, Hkv, d, seed)
    td = getattr(torch, c["dtype"])
    q = torch.from_numpy(Q).to("cuda", td).requires_grad_()
    k = torch.from_numpy(K).to("cuda", td).requires_grad_()
    v = torch.from_numpy(V).to("cuda", td).requires_grad_()
    od = None if c["out"] is None else getattr(torch, c["out"])
    o = jm.masked_attention_via_map(q, k, v, out_dtype=od, precision=precision, **c["kw"])
    Qr, Kr, Vr = (x.detach().float().cpu().numpy() for x in (q, k, v))
    do_t = torch.from_numpy(dO).to("cuda", o.dtype)
    O_ref, _, g_ref, _ = oracle(Qr, Kr, Vr, do_t.float().cpu().numpy(), c["kw"])
    out_name = str(o.dtype).replace("torch.", "")
    scale = A.kernel_scale(c["kw"].get("kernel_fn", A.default_kernel), d)
    fast = not A.use_precise(precision, scale, d)
    floor = Floor() if fast else None
    assert_close(o.detach().float().cpu().numpy(), O_ref, c["dtype"], "O", out_name, floor=floor)
    o.backward(do_t)
    for name, t, r in (("dQ", q, g_ref[0]), ("dK", k, g_ref[1]), ("dV", v, g_ref[2])):
        assert_close(t.grad.float().cpu().numpy(), r, c["dtype"], name, floor=floor)
    torch.cuda.synchronize()
    if floor is not None and floor.misses:
        run_draw(seed, precision="highest")
        floor.finish()


@pytest.mark.parametrize("seed", range(24))
def test_random_problem(seed):
    run_draw(seed)


# Draws of seeds 24-623 that failed the gate with bfloat16 dS (dK, dQ) and
# dO (dQ) operands, every one a bfloat16 threshold_kernel problem (now run in
# float32 arithmetic: precision None picks "highest" for threshold_kernel).
KNOWN_DRAWS = [25, 31, 94, 100, 118, 165, 196, 226, 231, 311, 332, 444, 478, 590]


@pytest.mark.parametrize("seed", KNOWN_DRAWS)
def test_known_draw(seed):
    run_draw(seed)


# The draws of seeds 624-1423 that missed the earlier, looser gate with the
# float16 operands: single 16-bit dV / dQ elements rounded one ulp off.
LATER_DRAWS = [647, 696, 976, 1060, 1067, 1073, 1120, 1193, 1201, 1246, 1271, 1288, 1414]


@pytest.mark.parametrize("seed", LATER_DRAWS)
def test_later_draw(seed):
    run_draw(seed)


# The one draw of a one-off 800-problem run (seeds 1424-2223) that missed the
# gate with split tiles at a largest weight of 1/8: cross attention onto 12
# keys, every weight about 1/12 (split tiles now start at 1/32).
SPLIT_DRAWS = [2120]


@pytest.mark.parametrize("seed", SPLIT_DRAWS)
def test_split_draw(seed):
    run_draw(seed)


# The one draw of a one-off 800-problem run (seeds 2224-3023) that misses the
# gate with split rows at 1/32: cross attention onto 56 keys (every weight
# about 1/56: no split row), two query heads per kv head, bfloat16 dV
# elements just above 1, where half a bfloat16 ulp (2^-8) leaves 1.5e-4 of the
# gate and the float16 rounding of 664 comparable terms exceeds it: 1.003x
# the gate, within the operands' bound.  Reported xfailed after "highest"
# meets the gate.
FLOOR_DRAWS = [2477]


@pytest.mark.parametrize("seed", FLOOR_DRAWS)
def test_floor_draw(seed):
    run_draw(seed)


def test_draws_cover_every_family():
    fams = {draw(s)["fam"] for s in range(24)}
    assert fams == set(FAMILIES)


def test_threshold_kernel_fp32():
    """threshold_kernel(t) through the float32 path, against the oracle at
    scale 1 (1e-5 gate), forward and backward, with a causal mask."""
    import jaxmodules_amd as jm
    from jaxmodules_amd import attention as A

    B, N, L, Hq, Hkv, d = 2, 150, 150, 4, 2, 64
    Q, K, V, dO = seeded_inputs(B, N, L, Hq, Hkv, d, 77)   # logits q.k of unit variance
    kw = dict(is_causal=True, block_size=32, kernel_fn=A.threshold_kernel(1.5))
    q, k, v = (torch.from_numpy(x).to("cuda").requires_grad_() for x in (Q, K, V))
    o = jm.masked_attention_via_map(q, k, v, **kw)
    O_ref, _, g_ref, _ = oracle(Q, K, V, dO, kw)
    assert_close(o.detach().cpu().numpy(), O_ref, "float32", "O")
    o.backward(torch.from_numpy(dO).to("cuda"))
    for name, t, r in (("dQ", q, g_ref[0]), ("dK", k, g_ref[1]), ("dV", v, g_ref[2])):
        assert_close(t.grad.cpu().numpy(), r, "float32", name)
