"""GPU parity: the HIP path (through the C ABI) against the fp64 oracle.

Inputs are seeded, rounded to the kernel dtype once, and the oracle runs on
those exact values, under the parity gate of tests/helpers.py (the north
star's 2e-3 + 2e-3 |b| for 16-bit O and gradients, 1e-5 for float32; half an
output ulp plus float32 accumulation where that is coarser).  A 16-bit case
whose default-path result misses the gate only within the float16 operands'
error bound (tests/helpers.py Floor) is run again with precision="highest",
which must meet the gate, and is then reported xfailed with its ratios.
"""
import math

import numpy as np
import pytest

from tests.helpers import Floor, assert_close, oracle, seeded_inputs

torch = pytest.importorskip("torch")

pytestmark = pytest.mark.gpu

DT = {"bfloat16": None, "float16": None, "float32": None}


def _tdt(name):
    return getattr(torch, name)


def run_case(shape, kw, dtype="bfloat16", seed=0, out_dtype=None, scaled=True, grads=True, precision=None):
    """One case against the oracle; a default-path miss within the float16
    operands' bound reruns the case at precision "highest" (which must pass)
    and then xfails."""
    import jaxmodules_amd as jm

    B, N, L, Hq, Hkv, d = shape
    Q, K, V, dO = seeded_inputs(B, N, L, Hq, Hkv, d, seed, scaled=scaled)
    td = _tdt(dtype)
    dev = "cuda"
    q = torch.from_numpy(Q).to(dev, td).requires_grad_(grads)
    k = torch.from_numpy(K).to(dev, td).requires_grad_(grads)
    v = torch.from_numpy(V).to(dev, td).requires_grad_(grads)
    od = None if out_dtype is None else _tdt(out_dtype)
    o = jm.masked_attention_via_map(q, k, v, out_dtype=od, precision=precision, **kw)
    assert o.dtype == (torch.float32 if od is None else od)
    # the oracle sees exactly the rounded inputs
    Qr, Kr, Vr = (x.detach().float().cpu().numpy() for x in (q, k, v))
    do_t = torch.from_numpy(dO).to(dev, o.dtype)
    dOr = do_t.float().cpu().numpy()
    O_ref, _, g_ref, _ = oracle(Qr, Kr, Vr, dOr, kw, grads=grads)
    out_name = str(o.dtype).replace("torch.", "")
    floor = Floor() if precision is None and dtype != "float32" else None
    tag = "" if precision is None else f"[{precision}] "
    assert_close(o.detach().float().cpu().numpy(), O_ref, dtype, tag + "O", out_name, floor=floor)
    if grads:
        o.backward(do_t)
        for name, t, r in (("dQ", q, g_ref[0]), ("dK", k, g_ref[1]), ("dV", v, g_ref[2])):
            assert t.grad.dtype == td
            assert_close(t.grad.float().cpu().numpy(), r, dtype, tag + name, floor=floor)
    torch.cuda.synchronize()
    if floor is not None and floor.misses:
        run_case(shape, kw, dtype, seed, out_dtype, scaled, grads, precision="highest")
        floor.finish()


CAUSAL = dict(is_causal=True)


def _docs(L, seed, mean=300, minlen=16):
    rng = np.random.default_rng(seed)
    lens = []
    while sum(lens) < L:
        lens.append(max(minlen, int(rng.geometric(1.0 / mean))))
    doc = np.repeat(np.arange(len(lens)), lens)[:L]
    return doc


def _block_sparse(nt, H, seed, density=0.25):
    rng = np.random.default_rng(seed)
    tbl = rng.random((H, nt, nt)) < density
    tbl[:, np.arange(nt), np.arange(nt)] = True
    return tbl


def test_cfg1_fp32_causal_forward():
    """BASELINE cfg1: fp32 [2,128,8,64] causal, block 32, forward at 1e-5."""
    run_case((2, 128, 128, 8, 8, 64), dict(is_causal=True, block_size=32), "float32",
             scaled=False, grads=False)


@pytest.mark.parametrize("d", [64, 128])
def test_fp32_masked_fwd_bwd(d):
    run_case((1, 200, 200, 2, 2, d), dict(mask_fn=lambda h, q, k: (q - k) % 5 != 2, block_size=40),
             "float32", scaled=False)


@pytest.mark.parametrize("dtype", ["bfloat16", "float16"])
@pytest.mark.parametrize("d", [64, 128])
def test_causal_fwd_bwd(dtype, d):
    run_case((2, 384, 384, 2, 2, d), dict(is_causal=True, block_size=128), dtype)


# head dimension 256: the float32 SIMT kernels for every input dtype (ragged
# lengths, grouped heads, a partial-tile mask, both output dtypes)
@pytest.mark.parametrize("dtype", ["bfloat16", "float16", "float32"])
def test_d256_causal_gqa_fwd_bwd(dtype):
    run_case((2, 300, 300, 4, 2, 256), dict(is_causal=True, block_size=128), dtype,
             scaled=dtype != "float32")


@pytest.mark.parametrize("dtype", ["bfloat16", "float16"])
def test_d256_masked_16bit_output(dtype):
    run_case((1, 200, 330, 2, 1, 256), dict(mask_fn=lambda h, q, k: (q + 3 * h - k) % 7 != 0,
                                            block_size=64), dtype, out_dtype=dtype, seed=3)


def test_full_attention_no_block_size():
    run_case((1, 256, 256, 2, 2, 128), {}, "bfloat16")


def test_sliding_window_cfg3_small():
    """cfg3 scaled down: (q>=k)&(q-k<=200) with window_size (200, 0) at block 128."""
    run_case((1, 1024, 1024, 2, 2, 128),
             dict(mask_fn=lambda b, h, q, k: (q >= k) & (q - k <= 200), window_size=(200, 0),
                  block_size=128), "bfloat16")


def test_window_changes_result():
    """A permissive mask with a narrow block window (attention.py:374-381)."""
    run_case((1, 640, 640, 2, 2, 64), dict(block_size=64, window_size=(64, 64)), "bfloat16")


def test_block_sparse_cfg4_small():
    """cfg4 scaled down: per-head random 128x128 tiles, diagonal on, causal inside it."""
    H, L = 4, 1024
    tbl = _block_sparse(L // 128, H, 7)
    mask = lambda b, h, q, k: tbl[h, q // 128, k // 128] & ((q // 128 != k // 128) | (q >= k))
    run_case((1, L, L, H, H, 64), dict(mask_fn=mask, block_size=128), "bfloat16")


def test_packed_documents_cfg5_small():
    L = 2048
    doc = _docs(L, 3)
    mask = lambda b, h, q, k: (doc[q] == doc[k]) & (q >= k)
    run_case((1, L, L, 2, 2, 128), dict(mask_fn=mask, block_size=128), "bfloat16")


def test_gqa():
    run_case((2, 256, 256, 4, 2, 128), dict(is_causal=True, block_size=64), "bfloat16")


@pytest.mark.parametrize("closed_form", [True, False])
def test_reference_benchmark_regime_small(closed_form):
    """check_attn.py's regime scaled down (its L >= 32768, period 2048, block
    8192): float16, one head, d = 64, unit-variance inputs, mask
    k % P == q % P and k <= q (check_attn.py:9-32), here P = 512, L = 4096,
    block 1024; the closed form (GPU tile map) and the plain lambda (host tracer).
    A key is attended by at most L / P queries, each with at most L / P keys,
    so a dV element is a sum of a few terms of size ~0.5 that often cancel: one
    element (key 890, a sum of 7 terms of up to 1.9 cancelling to 0.017) misses
    the 2e-3 absolute tolerance by 1.12x, within the float16 operands' bound
    (the float64 model of the design's roundings, tests/rounding_model.py,
    gives the kernel's value to the output ulp: tests/test_rounding_model.py).
    The same problem at precision "highest" meets the gate."""
    import jaxmodules_amd as jm
    from jaxmodules_amd import masks

    P, L, d = 512, 4096, 64
    mf = (masks.intersect(masks.same_residue(P), masks.causal()) if closed_form
          else (lambda b, h, q, k: (k <= q) & (k % P == q % P)))
    kw = dict(mask_fn=mf, block_size=1024)
    Q, K, V, dO = seeded_inputs(1, L, L, 1, 1, d, 21, scaled=False)
    Qr, Kr, Vr = (torch.from_numpy(x).to(torch.float16).double().numpy() for x in (Q, K, V))
    O_ref, _, g_ref, _ = oracle(Qr, Kr, Vr, dO, kw)
    floor = Floor()
    for precision in (None, "highest"):
        q, k, v = (torch.from_numpy(x).to("cuda", torch.float16).requires_grad_() for x in (Q, K, V))
        o = jm.masked_attention_via_map(q, k, v, precision=precision, **kw)
        fl = floor if precision is None else None
        assert_close(o.detach().double().cpu().numpy(), O_ref, "float16", f"{precision} O", "float32", floor=fl)
        o.backward(torch.from_numpy(dO).cuda())
        for name, t, r in (("dQ", q, g_ref[0]), ("dK", k, g_ref[1]), ("dV", v, g_ref[2])):
            assert_close(t.grad.double().cpu().numpy(), r, "float16", f"{precision} {name}", floor=fl)
        torch.cuda.synchronize()
    floor.finish()


def test_gqa_head_specific_mask():
    mask = lambda b, h, q, k: (q + 40 * h) >= k
    run_case((1, 256, 256, 4, 1, 64), dict(mask_fn=mask, block_size=64), "bfloat16")


def test_batch_specific_mask():
    mask = lambda b, h, q, k: (q // (37 + 11 * b)) == (k // (37 + 11 * b))
    run_case((3, 300, 300, 2, 2, 64), dict(mask_fn=mask, block_size=100), "bfloat16")


@pytest.mark.parametrize("dtype", ["bfloat16", "float32"])
def test_padding_ragged(dtype):
    """N=200, L=333, block 64: the reference pads to a block multiple (attention.py:426-437)."""
    run_case((2, 200, 333, 2, 2, 64), dict(is_causal=True, block_size=64), dtype,
             scaled=(dtype != "float32"))


def test_padding_tiny():
    """test_mapped_attention.py:1076-1112 shape: N=10, L=13, block 4."""
    run_case((1, 10, 13, 4, 4, 64), dict(mask_fn=lambda h, q, k: abs(q - k) <= 2, block_size=4),
             "float32", scaled=False)


def test_empty_rows_zero():
    mask = lambda b, h, q, k: (q > 100) & (k <= q)
    run_case((1, 256, 256, 2, 2, 128), dict(mask_fn=mask, block_size=128), "bfloat16")


def test_bf16_output_dtype():
    run_case((1, 256, 256, 2, 2, 128), dict(is_causal=True, block_size=128), "bfloat16",
             out_dtype="bfloat16")


def test_three_dim_inputs():
    import jaxmodules_amd as jm

    Q, K, V, dO = seeded_inputs(1, 96, 96, 2, 2, 64, 5, scaled=False)
    q, k, v = (torch.from_numpy(x[0]).cuda() for x in (Q, K, V))
    o = jm.masked_attention_via_map(q, k, v, is_causal=True, block_size=32)
    O_ref, _, _, _ = oracle(Q[0], K[0], V[0], None, dict(is_causal=True, block_size=32), grads=False)
    assert o.shape == (96, 2, 64)
    assert_close(o.cpu().numpy(), O_ref, "float32", "O")


def test_noncontiguous_inputs():
    import jaxmodules_amd as jm

    Q, K, V, _ = seeded_inputs(1, 128, 128, 2, 2, 64, 6)
    # [B, H, L, d] storage viewed as [B, L, H, d]
    q, k, v = (torch.from_numpy(x).cuda().to(torch.bfloat16).transpose(1, 2).contiguous().transpose(1, 2)
               for x in (Q, K, V))
    o = jm.masked_attention_via_map(q, k, v, is_causal=True)
    O_ref, _, _, _ = oracle(*(x.float().cpu().numpy() for x in (q, k, v)), None,
                            dict(is_causal=True), grads=False)
    assert_close(o.cpu().numpy(), O_ref, "bfloat16", "O")


def test_deterministic():
    """No atomics: two runs are bitwise identical."""
    import jaxmodules_amd as jm

    Q, K, V, dO = seeded_inputs(1, 512, 512, 4, 2, 128, 9)
    outs = []
    for _ in range(2):
        q, k, v = (torch.from_numpy(x).cuda().to(torch.bfloat16).requires_grad_() for x in (Q, K, V))
        o = jm.masked_attention_via_map(q, k, v, is_causal=True, block_size=128)
        o.backward(torch.from_numpy(dO).cuda())
        outs.append([o.detach(), q.grad, k.grad, v.grad])
    for a, b in zip(*outs):
        assert torch.equal(a, b)


@pytest.mark.parametrize("dtype", ["float32", "bfloat16"])
def test_reference_custom_kernel(dtype):
    """The reference's test_masked_attention_different_kernel
    (test_mapped_attention.py:1122-1144): kernel exp(q.k / (2 sqrt(d))) on
    N(0, 1) inputs of shape [8, 4, 16], here against the oracle at scale
    1 / (2 sqrt(d)), forward and backward; and, as there, the result differs
    from the default kernel's."""
    import jaxmodules_amd as jm

    def custom_kernel(q, k):
        return np.exp(np.dot(q, k) / (2 * np.sqrt(k.shape[-1])))

    N, Hq, d = 8, 4, 16
    rng = np.random.default_rng(42)
    Q, K, V, dO = (rng.standard_normal((N, Hq, d)).astype(np.float32) for _ in range(4))
    td = getattr(torch, dtype)
    q, k, v = (torch.from_numpy(x).to("cuda", td).requires_grad_() for x in (Q, K, V))
    o = jm.masked_attention_via_map(q, k, v, kernel_fn=custom_kernel)
    Qr, Kr, Vr = (x.detach().float().cpu().numpy() for x in (q, k, v))
    O_ref, _, g_ref, _ = oracle(Qr, Kr, Vr, dO, {}, scale=1 / (2 * math.sqrt(d)))
    assert_close(o.detach().float().cpu().numpy(), O_ref, dtype, "O", "float32")
    o.backward(torch.from_numpy(dO).to("cuda"))
    for name, t, r in (("dQ", q, g_ref[0]), ("dK", k, g_ref[1]), ("dV", v, g_ref[2])):
        assert_close(t.grad.float().cpu().numpy(), r, dtype, name)
    o_def = jm.masked_attention_via_map(q.detach(), k.detach(), v.detach())
    assert not torch.allclose(o.detach(), o_def, rtol=1e-2)


@pytest.mark.parametrize("causal", [True, False])
def test_residue_rewrite_gqa_and_layouts(causal):
    """The residue-class rewrite (attention._residue_rewrite) with grouped heads,
    bfloat16 inputs, a 16-bit output, 3-D inputs and both mask forms (with and
    without causal), against the oracle: the strided views carry the same
    attention as the original order."""
    import jaxmodules_amd as jm
    from jaxmodules_amd import masks

    P, L, Hq, Hkv, d = 16, 512, 4, 2, 64
    mf = masks.intersect(masks.same_residue(P), masks.causal()) if causal else masks.same_residue(P)
    kw = dict(mask_fn=mf, block_size=64)
    Q, K, V, dO = seeded_inputs(1, L, L, Hq, Hkv, d, 31)
    # dO rounded to bfloat16 once: the float32-output run and the bfloat16 one see the same values
    Qr, Kr, Vr, dO = (torch.from_numpy(x).to(torch.bfloat16).float().numpy() for x in (Q, K, V, dO))
    O_ref, _, g_ref, _ = oracle(Qr, Kr, Vr, dO, kw)
    floor = Floor()
    for three, od in ((False, None), (True, torch.bfloat16)):
        q, k, v = (torch.from_numpy(x[0] if three else x).to("cuda", torch.bfloat16).requires_grad_()
                   for x in (Q, K, V))
        o = jm.masked_attention_via_map(q, k, v, out_dtype=od, **kw)
        assert o.shape == q.shape and o.dtype == (od or torch.float32)
        sq = (lambda x: x[0]) if three else (lambda x: x)
        out_name = "bfloat16" if od is not None else "float32"
        assert_close(o.detach().float().cpu().numpy(), sq(np.asarray(O_ref)), "bfloat16", f"3d={three} O",
                     out_name, mag=sq(O_ref.mag), floor=floor)
        o.backward(torch.from_numpy(sq(dO)).to("cuda", o.dtype))
        for name, t, r in (("dQ", q, g_ref[0]), ("dK", k, g_ref[1]), ("dV", v, g_ref[2])):
            assert_close(t.grad.float().cpu().numpy(), sq(np.asarray(r)), "bfloat16", f"3d={three} {name}",
                         mag=sq(r.mag), floor=floor)
    torch.cuda.synchronize()
    floor.finish()
