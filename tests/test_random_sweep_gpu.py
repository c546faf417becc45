"""A seeded random sweep of problem shapes and masks: the HIP path against the
fp64 oracle under the parity gate of tests/helpers.py.  Each case draws batch
size, query/key lengths (1..400, often ragged), GQA layout, head dim
(16..128, padded to 64/128 by the host), dtype, block size, kernel function,
output dtype and one mask family: causal, none, an element window with the
reference's block window, packed documents, a per-head tile table, a
head-specific lambda, or cross lengths.  The draw is fixed by the seed, so
every run checks the same problems: seeds 0-23, the draws of a one-off
600-problem run (seeds 24-623) that failed the gate with the kernels' earlier
bfloat16 dS / dO operands (KNOWN_DRAWS), and the thirteen draws of two more
one-off runs (seeds 624-1423, the current kernels) that miss it (LATER_FLOOR).

threshold_kernel is a softmax with scale 1 instead of 1/sqrt(d), so its
draws see logits of unit variance (Q, K ~ N(0,1) d^-0.25), seven times
sharper than the default kernel's at d = 48."""
import numpy as np
import pytest

from tests.helpers import assert_close, oracle, seeded_inputs

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


def run_draw(seed):
    import jaxmodules_amd as jm

    c = draw(seed)
    B, N, L, Hq, Hkv, d = c["shape"]
    print(f"[sweep] seed={seed} {c['fam']} shape={c['shape']} dtype={c['dtype']} out={c['out']} "
          f"kw={ {k: v for k, v in c['kw'].items() if k != 'mask_fn'} }", flush=True)
    Q, K, V, dO = seeded_inputs(B, N, L, Hq, Hkv, d, seed)
    td = getattr(torch, c["dtype"])
    q = torch.from_numpy(Q).to("cuda", td).requires_grad_()
    k = torch.from_numpy(K).to("cuda", td).requires_grad_()
    v = torch.from_numpy(V).to("cuda", td).requires_grad_()
    od = None if c["out"] is None else getattr(torch, c["out"])
    o = jm.masked_attention_via_map(q, k, v, out_dtype=od, **c["kw"])
    Qr, Kr, Vr = (x.detach().float().cpu().numpy() for x in (q, k, v))
    do_t = torch.from_numpy(dO).to("cuda", o.dtype)
    O_ref, _, g_ref, _ = oracle(Qr, Kr, Vr, do_t.float().cpu().numpy(), c["kw"])
    out_name = str(o.dtype).replace("torch.", "")
    assert_close(o.detach().float().cpu().numpy(), O_ref, c["dtype"], "O", out_name)
    o.backward(do_t)
    for name, t, r in (("dQ", q, g_ref[0]), ("dK", k, g_ref[1]), ("dV", v, g_ref[2])):
        assert_close(t.grad.float().cpu().numpy(), r, c["dtype"], name)
    torch.cuda.synchronize()


@pytest.mark.parametrize("seed", range(24))
def test_random_problem(seed):
    run_draw(seed)


# Draws of seeds 24-623 that failed the gate with bfloat16 dS (dK, dQ) and
# dO (dQ) operands, every one a bfloat16 threshold_kernel problem.
KNOWN_DRAWS = [25, 31, 94, 100, 118, 165, 196, 226, 231, 311, 332, 444, 478, 590]


# With every operand in float16 (and O's weights summed as rounded), 11 of
# them pass; the other three exceed the gate in single elements of dK / dV
# whose sums of float16-rounded products cancel.  The CPU model of the
# kernels' roundings (tests/test_rounding_model.py) reproduces them: the
# floor of 16-bit matrix-core operands, not a kernel error.
FLOOR = {
    31: "1 dK element of 493056 at 1.007x the bound (float16 operand floor)",
    94: "1 dV element of 92160 at 1.004x the bound (float16 operand floor)",
    118: "dK/dV of 4 keys summed over 236 queries cancel to ~0.1 (54 of 3072 elements, "
         "1.5x; float16 operand floor)",
}


@pytest.mark.parametrize("seed", [pytest.param(s, marks=pytest.mark.xfail(strict=True, reason=FLOOR[s]))
                                  if s in FLOOR else s for s in KNOWN_DRAWS])
def test_known_draw(seed):
    run_draw(seed)


# The misses of the 800 draws of seeds 624-1423: one or two 16-bit output
# elements each, rounded one ulp off because the float32 sum of float16-rounded
# products lands past the rounding midpoint.  tests/test_rounding_model.py
# reproduces each ratio with the model of the kernels' roundings (draw 1120:
# the model's sum lies within 2e-6 of the midpoint).
LATER_FLOOR = {
    647: "1 dQ element of 199680 at 1.015x the bound (threshold_kernel; float16 operand floor)",
    696: "1 dV element of 188928 at 1.051x the bound (float16 operand floor)",
    976: "1 dV element of 247040 at 1.024x the bound (float16 operand floor)",
    1060: "1 dV element of 145920 at 1.026x the bound (threshold_kernel; float16 operand floor)",
    1067: "1 dV element of 124160 at 1.052x the bound (threshold_kernel; float16 operand floor)",
    1073: "2 dV elements of 112128 at up to 1.035x the bound (threshold_kernel; float16 operand floor)",
    1120: "1 dV element of 69120 at 1.017x the bound, its float32 sum at a rounding midpoint "
          "(threshold_kernel; float16 operand floor)",
    1193: "1 dV element of 199680 at 1.002x the bound (float16 operand floor)",
    1201: "1 dV element of 25920 at 1.013x the bound (float16 operand floor)",
    1246: "1 dV element of 21504 at 1.049x the bound (float16 operand floor)",
    1271: "2 float16 dV elements of 16768 at up to 1.302x the bound (float16 operand floor)",
    1288: "1 dV element of 67968 at 1.113x the bound (float16 operand floor)",
    1414: "1 dV element of 192000 at 1.026x the bound (threshold_kernel; float16 operand floor)",
}


@pytest.mark.parametrize("seed", [pytest.param(s, marks=pytest.mark.xfail(strict=True, reason=r))
                                  for s, r in sorted(LATER_FLOOR.items())])
def test_later_floor_draw(seed):
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
