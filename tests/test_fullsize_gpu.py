"""Parity at the BASELINE configurations' full sizes (GPU).

The fp64 CPU oracle cannot run at these sizes, so for a floating-point kernel
the check is a float64 torch reference on the GPU (dense masked softmax
attention, chunked over queries, every key), itself pinned to the oracle's
dense_forward / dense_backward on a slice small enough for the CPU, under the
same element-wise gate as the oracle tests (tests/helpers.py, with the
reference's own term magnitudes for the accumulation slack).  At the north
star's target shape and at cfg2 every KV head is checked element by element;
at the larger cfg3-cfg5 the first and the last.  Every head is further checked
through two identities that hold for any input, whatever the size:
  * sum_k dV[b, k, hk] = sum over the group's heads h and non-empty rows q of dO[b, q, h]
    (the attention weights of a row sum to one);
  * sum_k dK[b, k, hk] = 0  (sum_k dS[q, k] = 0 for every row).
Besides the five configurations through masked_attention_via_map: the target
shape with grouped heads (Hq=32, Hkv=8; dK and dV of a KV head sum over its
four query heads), and cfg4 as the BASELINE words it, create_block_mask ->
flex_attention (BlockMask.tile_map), on [B, H, L, E] views.  A configuration
whose default-path result misses the gate only within the float16 operands'
error bound (tests/helpers.py Floor) is run again at precision "highest"
(float32 arithmetic), whose sampled heads must meet the gate, and is then
reported xfailed with its ratios.
"""
import math

import numpy as np
import pytest

from tests.helpers import Floor, assert_close, magnitudes

torch = pytest.importorskip("torch")

pytestmark = pytest.mark.gpu


def _docs(L, seed, mean=2048, minlen=64):
    rng = np.random.default_rng(seed)
    lens = []
    while sum(lens) < L:
        lens.append(max(minlen, int(rng.geometric(1.0 / mean))))
    return np.repeat(np.arange(len(lens)), lens)[:L]


def config(name):
    """(B, L, Hq, Hkv, d, kwargs, numpy mask of (h, q[:,None], k[None,:]))."""
    if name == "cfg2":
        kw = dict(is_causal=True, block_size=128)
        return 4, 4096, 32, 32, 128, kw, lambda h, q, k: q >= k
    if name in ("target", "target_gqa"):   # the north star's shape, and with Hkv = 8
        kw = dict(is_causal=True, block_size=128)
        return 1, 8192, 32, 32 if name == "target" else 8, 128, kw, lambda h, q, k: q >= k
    if name == "cfg3":
        m = lambda b, h, q, k: (q >= k) & (q - k <= 512)
        kw = dict(mask_fn=m, window_size=(512, 0), block_size=128)
        return 2, 16384, 16, 16, 128, kw, lambda h, q, k: (q >= k) & (q - k <= 512)
    if name in ("cfg4", "cfg4_block_mask"):
        nt, H = 64, 32
        rng = np.random.default_rng(4)
        tbl = rng.random((H, nt, nt)) < 0.25
        tbl[:, np.arange(nt), np.arange(nt)] = True
        m = lambda b, h, q, k: tbl[h, q // 128, k // 128] & ((q // 128 != k // 128) | (q >= k))
        return 1, 8192, H, H, 64, dict(mask_fn=m, block_size=128), \
            lambda h, q, k: tbl[h, q // 128, k // 128] & ((q // 128 != k // 128) | (q >= k))
    if name == "cfg5":
        doc = _docs(32768, 5)
        m = lambda b, h, q, k: (doc[q] == doc[k]) & (q >= k)
        return 1, 32768, 8, 8, 128, dict(mask_fn=m, block_size=128), \
            lambda h, q, k: (doc[q] == doc[k]) & (q >= k)
    raise KeyError(name)


def reference_head(q, k, v, do, allowed_fn, h, chunk):
    """float64 dense reference for one (b, h): O, dQ, dK, dV and the sums of
    the magnitudes of their terms (the gate's accumulation slack, as
    tests/helpers.magnitudes); q/k/v/do [L, d] float64."""
    L, d = q.shape
    scale = 1.0 / math.sqrt(d)
    kidx = np.arange(k.shape[0])
    O, dQ, mO, mdQ = (torch.empty_like(q) for _ in range(4))
    dK, dV, mdK, mdV = (torch.zeros_like(k) for _ in range(4))
    ka, qa, va = k.abs(), q.abs(), v.abs()
    for q0 in range(0, L, chunk):
        qi = np.arange(q0, min(L, q0 + chunk))
        sl = slice(q0, q0 + len(qi))
        allowed = torch.from_numpy(np.asarray(allowed_fn(h, qi[:, None], kidx[None, :]), bool)).to(q.device)
        s = (q[sl] @ k.T) * scale
        s = s.masked_fill(~allowed, float("-inf"))
        m = s.amax(dim=1, keepdim=True)
        m = torch.where(torch.isfinite(m), m, torch.zeros_like(m))
        p = torch.exp(s - m).masked_fill(~allowed, 0.0)
        den = p.sum(dim=1, keepdim=True)
        p = p / torch.where(den > 0, den, torch.ones_like(den))
        g = do[sl]
        O[sl] = p @ v
        mO[sl] = p @ va
        dp = g @ v.T
        delta = (dp * p).sum(dim=1, keepdim=True)
        ds = p * (dp - delta)
        dQ[sl] = (ds @ k) * scale
        dK += (ds.T @ q[sl]) * scale
        dV += p.T @ g
        a = p * (dp.abs() + delta.abs())
        mdQ[sl] = (a @ ka) * scale
        mdK += (a.T @ qa[sl]) * scale
        mdV += p.T @ g.abs()
    return (O, dQ, dK, dV), (mO, mdQ, mdK, mdV)


def test_reference_head_matches_the_oracle():
    """The float64 GPU reference of this file against the oracle's dense
    functions (and tests/helpers.magnitudes) on CPU-sized slices of two of
    the masks above: the first 300 queries and keys of a causal and of a
    windowed head (a prefix of a causal row depends on the prefix alone)."""
    from oracle import attention_oracle as ao

    rng = np.random.default_rng(11)
    L, d = 300, 128
    for fn in (lambda h, q, k: q >= k, lambda h, q, k: (q >= k) & (q - k <= 70)):
        Q, K, V, dO = (rng.standard_normal((L, d)) * (d ** -0.25 if i < 3 else 1.0) for i in range(4))
        (O, dQ, dK, dV), mags = reference_head(*(torch.from_numpy(x).cuda() for x in (Q, K, V, dO)),
                                               fn, 0, 128)
        allowed = np.asarray(fn(0, np.arange(L)[:, None], np.arange(L)[None, :]), bool)[None, None]
        x4 = lambda x: x[None, :, None]  # noqa: E731  [L, d] -> [1, L, 1, d]
        ref_O, _ = ao.dense_forward(x4(Q), x4(K), x4(V), allowed)
        ref_g = ao.dense_backward(x4(Q), x4(K), x4(V), allowed, x4(dO))
        ref_m = magnitudes(x4(Q), x4(K), x4(V), allowed, x4(dO))
        for got, want in zip((O, dQ, dK, dV) + tuple(mags), (ref_O,) + tuple(ref_g) + tuple(ref_m)):
            np.testing.assert_allclose(got.cpu().numpy(), want[0, :, 0], rtol=1e-10, atol=1e-12)


def _run(name, q, k, v, do, kw, precision=None):
    """O [B, L, Hq, d] and the gradients, through masked_attention_via_map or,
    for cfg4_block_mask, create_block_mask + flex_attention on [B, H, L, E] views."""
    import jaxmodules_amd as jm

    if name != "cfg4_block_mask":
        o = jm.masked_attention_via_map(q, k, v, precision=precision, **kw)
        o.backward(do)
        return o
    from jaxmodules_amd.block_mask import create_block_mask

    B, L, H, _ = q.shape
    bm = create_block_mask(kw["mask_fn"], B, H, L, L, 128)
    o = jm.flex_attention(q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2), block_mask=bm,
                          precision=precision)
    o.backward(do.transpose(1, 2))
    return o.transpose(1, 2)


# configurations whose every KV head is checked element by element
ALL_HEADS = ("cfg2", "target", "target_gqa")


def _check_config(name, precision=None, floor=None):
    print(f"[fullsize] {name} precision={precision}", flush=True)
    B, L, Hq, Hkv, d, kw, allowed_fn = config(name)
    G = Hq // Hkv
    dev = torch.device("cuda")
    g = torch.Generator(device=dev)
    g.manual_seed(1234)
    f = d ** -0.25
    q = (torch.randn((B, L, Hq, d), generator=g, device=dev) * f).to(torch.bfloat16).requires_grad_()
    k = (torch.randn((B, L, Hkv, d), generator=g, device=dev) * f).to(torch.bfloat16).requires_grad_()
    v = (torch.randn((B, L, Hkv, d), generator=g, device=dev) * f).to(torch.bfloat16).requires_grad_()
    do = torch.randn((B, L, Hq, d), generator=g, device=dev)
    o = _run(name, q, k, v, do, kw, precision)
    torch.cuda.synchronize()
    assert o.dtype == torch.float32 and q.grad.dtype == torch.bfloat16

    # KV heads against the float64 reference: O and dQ of each query head of
    # the group, dK and dV summed over the group
    chunk = max(256, (1 << 27) // L)
    heads = [(b, hk) for b in range(B) for hk in range(Hkv)] if name in ALL_HEADS and precision is None \
        else [(0, 0), (B - 1, Hkv - 1)]
    for b, hk in heads:
        kf, vf = k[b, :, hk].detach().double(), v[b, :, hk].detach().double()
        dk_ref, dv_ref = torch.zeros_like(kf), torch.zeros_like(vf)
        mk_ref, mv_ref = torch.zeros_like(kf), torch.zeros_like(vf)
        for h in range(hk * G, (hk + 1) * G):
            with torch.no_grad():
                (O_r, dQ_r, dK_r, dV_r), (mO, mdQ, mdK, mdV) = reference_head(
                    q[b, :, h].detach().double(), kf, vf, do[b, :, h].double(), allowed_fn, h, chunk)
            dk_ref += dK_r
            dv_ref += dV_r
            mk_ref += mdK
            mv_ref += mdV
            for what, x, r, m in (("O", o[b, :, h], O_r, mO), ("dQ", q.grad[b, :, h], dQ_r, mdQ)):
                out_name = "float32" if what == "O" else "bfloat16"
                assert_close(x.detach().float().cpu().numpy(), r.cpu().numpy(), "bfloat16",
                             f"{name} b={b} h={h} {what}", out_name, mag=m.cpu().numpy(), floor=floor)
        for what, x, r, m in (("dK", k.grad[b, :, hk], dk_ref, mk_ref), ("dV", v.grad[b, :, hk], dv_ref, mv_ref)):
            assert_close(x.float().cpu().numpy(), r.cpu().numpy(), "bfloat16", f"{name} b={b} hk={hk} {what}",
                         mag=m.cpu().numpy(), floor=floor)

    # identities over every KV head (every configuration allows the diagonal,
    # so no row is empty)
    sum_dv = v.grad.float().sum(dim=1)                                # [B, Hkv, d]
    sum_do = do.sum(dim=1).reshape(B, Hkv, G, d).sum(2)
    scale_ = do.abs().sum(dim=1).reshape(B, Hkv, G, d).sum(2).clamp_min(1.0)
    rel = ((sum_dv - sum_do).abs() / scale_).max().item()
    sum_dk = k.grad.float().sum(dim=1)
    scale_k = k.grad.float().abs().sum(dim=1).clamp_min(1e-6)
    relk = (sum_dk.abs() / scale_k).max().item()
    print(f"[fullsize] {name}: identity deviations dV {rel:.3g}, dK {relk:.3g}", flush=True)
    assert rel < 5e-4, f"{name}: sum_k dV vs sum_q dO, max relative deviation {rel:.3g}"
    assert relk < 5e-3, f"{name}: sum_k dK should vanish, max relative {relk:.3g}"


@pytest.mark.parametrize("name", ["cfg2", "cfg3", "cfg4", "cfg4_block_mask", "cfg5", "target",
                                  "target_gqa"])
def test_baseline_config_full_size(name):
    floor = Floor()
    _check_config(name, floor=floor)
    if floor.misses:
        torch.cuda.empty_cache()
        _check_config(name, precision="highest")
        floor.finish()


def _check_attn_regime(precision, floor):
    import jaxmodules_amd as jm
    from jaxmodules_amd import masks

    L, d, P = 131072, 64, 2048
    print(f"[fullsize] check_attn regime precision={precision}", flush=True)
    dev = torch.device("cuda")
    g = torch.Generator(device=dev)
    g.manual_seed(42)
    q, k, v = (torch.randn((1, L, 1, d), generator=g, device=dev).to(torch.float16).requires_grad_()
               for _ in range(3))
    do = torch.randn((1, L, 1, d), generator=g, device=dev)
    kw = dict(mask_fn=masks.intersect(masks.same_residue(P), masks.causal()), block_size=8192)
    o = jm.masked_attention_via_map(q, k, v, precision=precision, **kw)
    o.backward(do)
    torch.cuda.synchronize()
    qf, kf, vf, dof = (t[0, :, 0].detach().double() for t in (q, k, v, do))
    scale = 1.0 / math.sqrt(d)
    kidx = torch.arange(L, device=dev)
    O_r, dQ_r, mO, mdQ = (torch.empty_like(qf) for _ in range(4))
    dK_r, dV_r, mdK, mdV = (torch.zeros_like(kf) for _ in range(4))
    chunk = 1024
    with torch.no_grad():
        for q0 in range(0, L, chunk):
            sl = slice(q0, q0 + chunk)
            qi = kidx[sl, None]
            allowed = ((qi - kidx[None, :]) % P == 0) & (qi >= kidx[None, :])
            s = (qf[sl] @ kf.T) * scale
            s = s.masked_fill(~allowed, float("-inf"))
            p = torch.softmax(s, dim=1)
            gq = dof[sl]
            O_r[sl] = p @ vf
            mO[sl] = p @ vf.abs()
            dp = gq @ vf.T
            delta = (dp * p).sum(dim=1, keepdim=True)
            ds = p * (dp - delta)
            dQ_r[sl] = (ds @ kf) * scale
            dK_r += (ds.T @ qf[sl]) * scale
            dV_r += p.T @ gq
            a = p * (dp.abs() + delta.abs())
            mdQ[sl] = (a @ kf.abs()) * scale
            mdK += (a.T @ qf[sl].abs()) * scale
            mdV += p.T @ gq.abs()
    for what, x, r, m, out in (("O", o[0, :, 0], O_r, mO, "float32"), ("dQ", q.grad[0, :, 0], dQ_r, mdQ, None),
                               ("dK", k.grad[0, :, 0], dK_r, mdK, None), ("dV", v.grad[0, :, 0], dV_r, mdV, None)):
        assert_close(x.detach().double().cpu().numpy(), r.cpu().numpy(), "float16", f"check_attn {what}", out,
                     mag=m.cpu().numpy(), floor=floor)


def test_reference_benchmark_regime_full_size():
    """The reference's own benchmark (check_attn.py:177-327) at its largest
    length: float16, B = 1, one head, d = 64, L = 131072, unit-variance inputs,
    block 8192, mask k % 2048 == q % 2048 and k <= q (check_attn.py:9-32),
    given in closed form so that its tile map is built on the GPU.  Every row,
    forward and backward, against a float64 dense reference on the GPU (the
    mask evaluated with torch there).  As in the scaled-down test, dV elements
    are sums of a few cancelling terms, and a few of 8.4 million miss the 2e-3
    absolute tolerance within the float16 operands' bound (tests/helpers.py
    Floor; tests/test_rounding_model.py reproduces such misses with the model
    of the design's roundings); at precision "highest" every element meets the
    gate."""
    floor = Floor()
    _check_attn_regime(None, floor)
    if floor.misses:
        torch.cuda.empty_cache()
        _check_attn_regime("highest", None)
        floor.finish()
