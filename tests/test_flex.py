"""flex_attention over BlockMask (attention.py:456-692) and head dimensions
other than 64, 128 and 256.

CPU: the reference's argument checks and exception types.
GPU: the HIP path against the fp64 oracle on the mask the block mask stands
for (``materialize_mask``, pinned in test_block_mask.py), under the parity gate
(1e-5 for float32, 2e-3 + 2e-3 |b| for 16-bit inputs); the reference tests'
shapes (test_attention.py:17-118: B=2, H=4, L=8, E=16, block 4) also against
torch's own CPU flex_attention at the reference tests' tolerance (1e-5).
"""
import math

import numpy as np
import pytest

from jaxmodules_amd.block_mask import BlockMask, create_block_mask
from oracle import attention_oracle as ao
from tests.helpers import Floor, Ref, assert_close, magnitudes

torch = pytest.importorskip("torch")

# the reference tests' masks (test_attention.py:77-95)
MASKS = {
    "causal": lambda b, h, q, k: q >= k,
    "sliding_window": lambda b, h, q, k: abs(q - k) <= 2,
    "alternating": lambda b, h, q, k: (q + k) % 2 == 0,
    "batch_head_sliding": lambda b, h, q, k: abs(q - k) <= b + h,
}


# --- CPU: argument checks -------------------------------------------------------


def _t(*shape):
    return torch.zeros(shape)


def test_flex_argument_checks():
    import jaxmodules_amd as jm

    q, k = _t(2, 4, 8, 16), _t(2, 4, 8, 16)
    with pytest.raises(NotImplementedError):
        jm.flex_attention(q, k, k, return_lse=True)
    with pytest.raises(AssertionError):
        jm.flex_attention(q, _t(2, 4, 8, 8), k)                  # E mismatch
    with pytest.raises(AssertionError):
        jm.flex_attention(q, _t(1, 4, 8, 16), _t(1, 4, 8, 16))   # B mismatch
    with pytest.raises(AssertionError):
        jm.flex_attention(q, k, _t(2, 4, 9, 16))                 # S mismatch
    with pytest.raises(AssertionError):
        jm.flex_attention(q, k, _t(2, 2, 8, 16))                 # Hv != Hkv
    with pytest.raises(AssertionError):
        jm.flex_attention(q, _t(2, 2, 8, 16), _t(2, 2, 8, 16))   # GQA without enable_gqa
    with pytest.raises(AssertionError):
        jm.flex_attention(_t(2, 3, 8, 16), _t(2, 2, 8, 16), _t(2, 2, 8, 16), enable_gqa=True)
    bm = BlockMask.causal_mask(2, 4, 8, 8, 4)
    with pytest.raises(AssertionError):
        jm.flex_attention(_t(2, 4, 12, 16), _t(2, 4, 12, 16), _t(2, 4, 12, 16), block_mask=bm)
    with pytest.raises(NotImplementedError):
        jm.flex_attention(q, k, k, score_mod=lambda s, b, h, i, j: s)
    with pytest.raises(NotImplementedError):
        jm.flex_attention(q, k, _t(2, 4, 8, 32))                 # Ev != E
    with pytest.raises(RuntimeError):
        jm.flex_attention(q, k, k)                               # CPU tensors: no CPU path
    # the slow variant accepts GQA without enable_gqa, and ignores return_lse
    with pytest.raises(RuntimeError):
        jm.flex_attention_slow(q, _t(2, 2, 8, 16), _t(2, 2, 8, 16), return_lse=True)


def test_tile_map_cache_is_per_head_layout():
    """Regression: the no-mask tile map was cached per (L, S) only, so a GQA
    call after a non-GQA call of the same lengths reused launch orders laid
    out for the other head count (items decoding to batches past B)."""
    from jaxmodules_amd import attention as A

    A.clear_cache()
    tm1 = A._block_mask_tiles(None, 2, 4, 4, 8, 8)
    tm2 = A._block_mask_tiles(None, 2, 4, 2, 8, 8)
    assert tm1 is not tm2 and (tm1.Hkv, tm2.Hkv) == (4, 2)
    kv = tm2.kv_order[tm2.kv_order >= 0]
    assert sorted(kv.tolist()) == list(range(2 * 2 * tm2.nkt))
    bm = create_block_mask(MASKS["causal"], 1, 1, 8, 8, 4)
    assert A._block_mask_tiles(bm, 2, 4, 4, 8, 8) is not A._block_mask_tiles(bm, 2, 4, 2, 8, 8)
    # a map traced for another shape is refused before any kernel call
    q, k = torch.zeros(2, 8, 4, 64), torch.zeros(2, 8, 2, 64)
    A._check_map(tm2, q, k)
    with pytest.raises(ValueError):
        A._check_map(tm1, q, k)
    with pytest.raises(ValueError):
        A._check_map(tm2, torch.zeros(1, 8, 4, 64), torch.zeros(1, 8, 2, 64))


# --- GPU --------------------------------------------------------------------------


def _oracle(q, k, v, allowed, scale, do=None):
    """fp64 O and grads for [B, H, L, E] float32 numpy inputs; allowed [B|1, Hq|1, L, S]."""
    Q, K, V = (np.swapaxes(x, 1, 2) for x in (q, k, v))
    B, L, Hq, _ = Q.shape
    al = np.broadcast_to(allowed, (B, Hq, L, K.shape[1]))
    O, _ = ao.dense_forward(Q, K, V, al, scale=scale)
    mags = magnitudes(Q, K, V, al, None if do is None else np.swapaxes(do, 1, 2), scale)
    g = None
    if do is not None:
        g = tuple(Ref(np.swapaxes(x, 1, 2), np.swapaxes(m, 1, 2))
                  for x, m in zip(ao.dense_backward(Q, K, V, al, np.swapaxes(do, 1, 2), scale=scale), mags[1:]))
    return Ref(np.swapaxes(O, 1, 2), np.swapaxes(mags[0], 1, 2)), g


def _inputs(shape_q, shape_kv, seed, dtype, scaled=True):
    rng = np.random.default_rng(seed)
    E = shape_q[-1]
    f = E ** -0.25 if scaled else 1.0
    mk = lambda s: torch.from_numpy((rng.standard_normal(s) * f).astype(np.float32)).to("cuda", dtype)
    q, k, v = mk(shape_q), mk(shape_kv), mk(shape_kv)
    do = torch.from_numpy(rng.standard_normal(shape_q).astype(np.float32)).to("cuda")
    return q, k, v, do


def _check(q, k, v, do, allowed, scale, dtype_name, grads=True, **kw):
    """flex (or ``fn``) against the oracle; a default-path miss within the
    float16 operands' bound (tests/helpers.py Floor) reruns the case at
    precision "highest", which must meet the gate, and then xfails."""
    import jaxmodules_amd as jm
    from jaxmodules_amd import attention as A

    fn = kw.pop("fn", jm.flex_attention)
    precision = kw.pop("precision", None)
    qg, kg, vg = (x.clone().requires_grad_(grads) for x in (q, k, v))
    o = fn(qg, kg, vg, scale=scale, precision=precision, **kw)
    assert o.shape == q.shape and o.dtype == torch.float32
    qn, kn, vn = (x.float().cpu().numpy() for x in (q, k, v))
    s = 1.0 / math.sqrt(q.shape[-1]) if scale is None else scale
    O, g = _oracle(qn, kn, vn, allowed, s, do.cpu().numpy() if grads else None)
    fast = dtype_name != "float32" and not A.use_precise(precision, s, q.shape[-1])
    floor = Floor() if fast else None
    assert_close(o.detach().cpu().numpy(), O, dtype_name, "O", "float32", floor=floor)
    if grads:
        o.backward(do)
        for name, t, r in (("dQ", qg, g[0]), ("dK", kg, g[1]), ("dV", vg, g[2])):
            assert t.grad.shape == t.shape and t.grad.dtype == t.dtype
            assert_close(t.grad.float().cpu().numpy(), r, dtype_name, name, floor=floor)
    if floor is not None and floor.misses:
        _check(q, k, v, do, allowed, scale, dtype_name, grads, fn=fn, precision="highest", **kw)
        floor.finish()
    return o


@pytest.mark.gpu
def test_flex_basic_no_mask():
    """test_attention.py:17-38 shapes (E=16, zero-padded to 64 for the kernels)."""
    q, k, v, do = _inputs((2, 4, 8, 16), (2, 4, 8, 16), 0, torch.float32, scaled=False)
    o = _check(q, k, v, do, np.ones((1, 1, 8, 8), bool), None, "float32")
    tfa = pytest.importorskip("torch.nn.attention.flex_attention")
    ref = tfa.flex_attention(q.cpu(), k.cpu(), v.cpu())
    assert np.allclose(o.detach().cpu().numpy(), ref.numpy(), rtol=1e-5, atol=1e-5)


@pytest.mark.gpu
def test_flex_gqa():
    """test_attention.py:41-63: Hq=4, Hkv=2, enable_gqa."""
    q, k, v, do = _inputs((2, 4, 8, 16), (2, 2, 8, 16), 1, torch.float32, scaled=False)
    o = _check(q, k, v, do, np.ones((1, 1, 8, 8), bool), None, "float32", enable_gqa=True)
    tfa = pytest.importorskip("torch.nn.attention.flex_attention")
    ref = tfa.flex_attention(q.cpu(), k.cpu(), v.cpu(), enable_gqa=True)
    assert np.allclose(o.detach().cpu().numpy(), ref.numpy(), rtol=1e-5, atol=1e-5)


@pytest.mark.gpu
@pytest.mark.parametrize("name", sorted(MASKS))
def test_flex_reference_block_masks(name):
    """test_attention.py:66-117: four masks, block 4, against the oracle and torch."""
    B, H, L, E = 2, 4, 8, 16
    fn = MASKS[name]
    q, k, v, do = _inputs((B, H, L, E), (B, H, L, E), 2, torch.float32, scaled=False)
    bm = create_block_mask(fn, B, H, L, L, 4)
    allowed = bm.materialize_mask().astype(bool)
    o = _check(q, k, v, do, allowed, None, "float32", block_mask=bm)
    tfa = pytest.importorskip("torch.nn.attention.flex_attention")
    tbm = tfa.create_block_mask(fn, B, H, L, L, device="cpu", BLOCK_SIZE=4, _compile=False)
    ref = tfa.flex_attention(q.cpu(), k.cpu(), v.cpu(), block_mask=tbm)
    assert np.allclose(o.detach().cpu().numpy(), ref.numpy(), rtol=1e-5, atol=1e-5)


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", ["bfloat16", "float16"])
def test_flex_16bit_block_sparse(dtype):
    """bf16/fp16, E=128, block 64, a per-head random block table with causal
    diagonal tiles, GQA 4:2, broadcast over the batch."""
    B, Hq, Hkv, L, E = 2, 4, 2, 512, 128
    rng = np.random.default_rng(7)
    tbl = rng.random((Hq, L // 64, L // 64)) < 0.4
    tbl[:, np.arange(L // 64), np.arange(L // 64)] = True
    fn = lambda b, h, q, k: tbl[h, q // 64, k // 64] & ((q // 64 != k // 64) | (q >= k))
    bm = create_block_mask(fn, 1, Hq, L, L, 64)
    q, k, v, do = _inputs((B, Hq, L, E), (B, Hkv, L, E), 3, getattr(torch, dtype))
    # partial tiles are the diagonal ones, whose elements do not depend on the head,
    # so the KV-head element rule of flex_attention gives materialize_mask's mask
    allowed = bm.materialize_mask().astype(bool)
    _check(q, k, v, do, allowed, None, dtype, block_mask=bm, enable_gqa=True)


@pytest.mark.gpu
def test_flex_causal_equals_masked_attention():
    """A causal BlockMask at block 128 is the same tile map as is_causal: the
    two entry points give bitwise equal outputs and gradients."""
    import jaxmodules_amd as jm

    B, H, L, E = 1, 4, 384, 128
    q, k, v, do = _inputs((B, H, L, E), (B, H, L, E), 4, torch.bfloat16)
    a = [x.clone().requires_grad_() for x in (q, k, v)]
    o1 = jm.flex_attention(*a, block_mask=create_block_mask(MASKS["causal"], 1, 1, L, L, 128))
    o1.backward(do)
    b = [x.transpose(1, 2).contiguous().requires_grad_() for x in (q, k, v)]
    o2 = jm.masked_attention_via_map(*b, is_causal=True, block_size=128)
    o2.backward(do.transpose(1, 2))
    assert torch.equal(o1, o2.transpose(1, 2))
    for x, y in zip(a, b):
        assert torch.equal(x.grad, y.grad.transpose(1, 2))
    assert o1.is_contiguous()


@pytest.mark.gpu
@pytest.mark.parametrize("scale", [0.3, -0.2, 0.0])
def test_flex_explicit_scale(scale):
    """Any finite scale (negative: sign folded into Q; zero: uniform weights)."""
    q, k, v, do = _inputs((1, 2, 96, 64), (1, 2, 96, 64), 5, torch.float32, scaled=False)
    bm = create_block_mask(MASKS["causal"], 1, 1, 96, 96, 32)
    _check(q, k, v, do, bm.materialize_mask().astype(bool), scale, "float32", block_mask=bm)


@pytest.mark.gpu
def test_flex_slow_evaluates_elements_with_query_head():
    """flex_attention_slow reads partial-tile elements with the query head
    (materialize_mask); flex_attention with the KV head (attention.py:561-575)."""
    import jaxmodules_amd as jm

    B, Hq, Hkv, L, E = 1, 4, 2, 64, 64
    fn = lambda b, h, q, k: (q + 8 * h) >= k
    bm = create_block_mask(fn, B, Hq, L, L, 16)
    q, k, v, do = _inputs((B, Hq, L, E), (B, Hkv, L, E), 6, torch.float32, scaled=False)
    _check(q, k, v, do, bm.materialize_mask().astype(bool), None, "float32", block_mask=bm,
           fn=jm.flex_attention_slow)
    tm = bm.tile_map(B, Hq, Hkv)                                    # KV-head elements
    _check(q, k, v, do, np.broadcast_to(tm.dense(), (B, Hq, L, L)), None, "float32", block_mask=bm,
           enable_gqa=True)


@pytest.mark.gpu
@pytest.mark.parametrize("d", [16, 32, 96, 160, 200, 384, 512])
def test_masked_attention_padded_head_dim(d):
    """Head dimensions other than 64/128/256/512 (zero-padded on the GPU to the
    next of the four; d > 128 runs on the float32 SIMT kernels), fwd + bwd."""
    import jaxmodules_amd as jm
    from tests.helpers import oracle, seeded_inputs

    kw = dict(mask_fn=lambda h, q, k: (q - k) % 4 != 1, block_size=32)
    Q, K, V, dO = seeded_inputs(1, 96, 96, 4, 2, d, 9)
    floor = Floor()
    for dt, name in ((torch.float32, "float32"), (torch.bfloat16, "bfloat16")):
        q, k, v = (torch.from_numpy(x).to("cuda", dt).requires_grad_() for x in (Q, K, V))
        o = jm.masked_attention_via_map(q, k, v, **kw)
        assert o.shape == (1, 96, 4, d)
        Qr, Kr, Vr = (x.detach().float().cpu().numpy() for x in (q, k, v))
        O, _, g, _ = oracle(Qr, Kr, Vr, dO, kw)
        fl = floor if name != "float32" and d <= 128 else None   # d > 128: float32 SIMT kernels
        assert_close(o.detach().cpu().numpy(), O, name, f"d={d} {name} O", "float32", floor=fl)
        o.backward(torch.from_numpy(dO).cuda())
        for nm, t, r in (("dQ", q, g[0]), ("dK", k, g[1]), ("dV", v, g[2])):
            assert_close(t.grad.float().cpu().numpy(), r, name, f"d={d} {name} {nm}", floor=fl)
    floor.finish()
