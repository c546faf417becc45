"""The GPU tile-map classifier (mattn_tilemap_classify / mattn_tilemap_bits)
against the host tracer: for masks in closed form both must produce the same
TileMap array for array (lists, mask numbering, bits, launch orders, pair
count), and attention through either map must agree bitwise.

The host tracer is itself pinned against the fp64 oracle's effective mask
(tests/test_oracle.py, tests/test_golden.py), so equality here carries that
pin over to the device path.
"""
import time

import numpy as np
import pytest

torch = pytest.importorskip("torch")

from jaxmodules_amd import attention as A          # noqa: E402
from jaxmodules_amd import blockmap as bmap         # noqa: E402
from jaxmodules_amd import masks                    # noqa: E402

pytestmark = pytest.mark.gpu

DEV = "cuda:0"


def assert_same_map(a: bmap.TileMap, b: bmap.TileMap):
    for f in ("B", "Hq", "Hkv", "Lq", "Lk", "map_b", "map_h", "nqt", "nkt", "pairs", "n_full",
              "n_partial"):
        assert getattr(a, f) == getattr(b, f), f
    for f in ("row_ptr", "row_ent", "col_ptr", "col_ent", "col_row", "row_bits", "col_bits",
              "q_order", "kv_order", "kv_desc"):
        x, y = getattr(a, f), getattr(b, f)
        assert x.shape == y.shape and x.dtype == y.dtype, (f, x.shape, y.shape, x.dtype, y.dtype)
        assert np.array_equal(x, y), f


def both(shape_q, shape_k, **kw):
    plan = bmap.make_plan(shape_q, shape_k, shape_k, **kw)
    t0 = time.perf_counter()
    host = bmap.trace(plan)
    th = time.perf_counter() - t0
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    dev = bmap.device_trace(plan, DEV)
    td = time.perf_counter() - t0
    print(f"host {th:.3f} s, device {td:.3f} s, nnz {host.nnz}, masks {host.n_masks}", flush=True)
    return host, dev


def _docs(L, seed, mean=300, minlen=16):
    rng = np.random.default_rng(seed)
    lens = []
    while sum(lens) < L:
        lens.append(max(minlen, int(rng.geometric(1.0 / mean))))
    return np.repeat(np.arange(len(lens)), lens)[:L]


CASES = {
    "causal": (((2, 1000, 4, 64), (2, 1000, 4, 64)), dict(is_causal=True, block_size=40)),
    "none_padded": (((1, 200, 2, 64), (1, 333, 2, 64)), dict(block_size=16)),
    "none_single_block": (((1, 256, 2, 64), (1, 512, 2, 64)), dict()),
    "window_clamped": (((2, 4096, 2, 64), (2, 4096, 2, 64)),
                       dict(mask_fn=masks.intersect(masks.causal(), masks.window(300, 0)),
                            window_size=(300, 0), block_size=128)),
    "window_small_blocks": (((1, 1000, 2, 64), (1, 1000, 2, 64)),
                            dict(mask_fn=masks.window(70, 30), window_size=(70, 30), block_size=25)),
    "bidirectional": (((1, 2000, 2, 64), (1, 2000, 2, 64)), dict(mask_fn=masks.window(64, 64))),
    "docs_causal": (((1, 8192, 2, 64), (1, 8192, 2, 64)),
                    dict(mask_fn=masks.intersect(masks.documents(_docs(8192, 1)), masks.causal()),
                         block_size=128)),
    "docs_per_batch": (((3, 1500, 2, 64), (3, 1500, 2, 64)),
                       dict(mask_fn=masks.documents(np.stack([_docs(1500, s) for s in range(3)])),
                            block_size=100)),
    "cross_docs": (((2, 300, 2, 64), (2, 1000, 2, 64)),
                   dict(mask_fn=masks.documents(np.arange(300) // 40, np.arange(1000) // 133),
                        block_size=100)),
    # the reference benchmark's strided mask (check_attn.py:9-32), scaled down
    "residue_causal": (((1, 8192, 1, 64), (1, 8192, 1, 64)),
                       dict(mask_fn=masks.intersect(masks.same_residue(1024), masks.causal()),
                            block_size=1024)),
    "residue_period_96": (((1, 1000, 2, 64), (1, 1000, 2, 64)),
                          dict(mask_fn=masks.intersect(masks.same_residue(96), masks.window(500, 30)),
                               block_size=100)),
    "residue_period_3_docs": (((2, 900, 2, 64), (2, 900, 2, 64)),
                              dict(mask_fn=masks.intersect(masks.same_residue(3),
                                                           masks.documents(_docs(900, 4)),
                                                           masks.causal()),
                                   block_size=90)),
}


def _table_case():
    rng = np.random.default_rng(7)
    H, nt = 4, 16
    tbl = (rng.random((H, nt, nt)) < 0.3).astype(np.uint8)
    tbl[:, np.arange(nt), np.arange(nt)] = 2            # diagonal: causal inside the tile
    return ((1, 2048, H, 64), (1, 2048, H, 64)), dict(
        mask_fn=masks.intersect(masks.tile_table(tbl), masks.causal()), block_size=128)


def _table_docs_case():
    rng = np.random.default_rng(8)
    B, H, nt = 2, 3, 10
    tbl = rng.integers(0, 3, size=(B, H, nt, nt)).astype(np.uint8)
    docs = np.stack([_docs(1200, 10 + b, mean=200) for b in range(B)])
    return ((B, 1200, H, 64), (B, 1200, H, 64)), dict(
        mask_fn=masks.intersect(masks.tile_table(tbl), masks.documents(docs), masks.window(500, None)),
        block_size=60)


CASES["table_per_head"] = _table_case()
CASES["table_docs_window"] = _table_docs_case()


@pytest.mark.parametrize("name", sorted(CASES))
def test_device_map_equals_host(name):
    (sq, sk), kw = CASES[name]
    host, dev = both(sq, sk, **kw)
    assert_same_map(host, dev)


def test_gqa_map_dims():
    (sq, sk), kw = _table_case()
    host, dev = both(sq, (1, 2048, 2, 64), **kw)     # Hkv = 2 for Hq = 4
    assert_same_map(host, dev)
    assert dev.map_h == 4


def test_mask_function_equals_lambda_map():
    """A masks.* function and the equivalent plain lambda trace to the same map
    (the lambda on the host, the closed form on the GPU)."""
    doc = _docs(4096, 3)
    plan_l = bmap.make_plan((1, 4096, 2, 64), (1, 4096, 2, 64), (1, 4096, 2, 64),
                            mask_fn=lambda b, h, q, k: (doc[q] == doc[k]) & (q >= k), block_size=128)
    plan_m = bmap.make_plan((1, 4096, 2, 64), (1, 4096, 2, 64), (1, 4096, 2, 64),
                            mask_fn=masks.intersect(masks.documents(doc), masks.causal()),
                            block_size=128)
    assert_same_map(bmap.trace(plan_l), bmap.device_trace(plan_m, DEV))


@pytest.mark.parametrize("cfg", ["cfg3", "cfg4", "cfg5"])
def test_fullsize_configs(cfg):
    """BASELINE configs 3-5 written as closed-form masks: same map as the host
    trace of the configs' lambdas (the ones bench.py and the full-size tests use)."""
    import bench

    B, L, H, _, d, kw, _ = bench.workload(cfg)
    shape = (B, L, H, d)
    plan = bmap.make_plan(shape, shape, shape, **kw)
    t0 = time.perf_counter()
    host = bmap.trace(plan)
    th = time.perf_counter() - t0
    kw2 = dict(kw)
    kw2["mask_fn"] = bench.closed_form_mask(cfg)
    plan2 = bmap.make_plan(shape, shape, shape, **kw2)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    dev = bmap.device_trace(plan2, DEV)
    td = time.perf_counter() - t0
    print(f"{cfg}: host {th:.2f} s, device {td:.3f} s", flush=True)
    assert_same_map(host, dev)


def test_attention_through_device_map_bitwise():
    """masked_attention_via_map with a closed-form mask (device map) equals the
    same call with the equivalent lambda (host map), forward and backward."""
    doc = _docs(1024, 4, mean=200)
    torch.manual_seed(0)
    q, k, v = (torch.randn(2, 1024, 4, 128, device=DEV, dtype=torch.bfloat16) for _ in range(3))
    do = torch.randn(2, 1024, 4, 128, device=DEV)
    outs = []
    for mf in (lambda b, h, qi, ki: (doc[qi] == doc[ki]) & (qi >= ki),
               masks.intersect(masks.documents(doc), masks.causal())):
        A.clear_cache()
        qq, kk, vv = (t.clone().requires_grad_() for t in (q, k, v))
        o = A.masked_attention_via_map(qq, kk, vv, mask_fn=mf, block_size=128)
        o.backward(do)
        outs.append([o.detach(), qq.grad, kk.grad, vv.grad])
    for x, y in zip(*outs):
        assert torch.equal(x, y)


def test_causal_call_uses_device_map(monkeypatch):
    """is_causal calls on the GPU are classified on the device (the host tracer
    is not called) and cached."""
    A.clear_cache()
    q = torch.randn(1, 512, 2, 64, device=DEV, dtype=torch.bfloat16)

    def no_host_trace(plan):
        raise AssertionError("host tracer called for a closed-form mask on the GPU")

    monkeypatch.setattr(bmap, "trace", no_host_trace)
    A.masked_attention_via_map(q, q, q, is_causal=True, block_size=64)
    monkeypatch.undo()
    plan, tm = A.trace_call((1, 512, 2, 64), (1, 512, 2, 64), (1, 512, 2, 64), is_causal=True,
                            block_size=64)
    assert_same_map(tm, bmap.trace(plan))


def test_bits_verify_flags_a_wrong_mask():
    """mattn_tilemap_bits in verify mode reports a mask that differs from the
    tile's (the check device_trace relies on against hash collisions)."""
    import ctypes

    from jaxmodules_amd import _lib

    lib = _lib.load()
    ms = _lib.MattnMaskspec(causal=1, win_left=-1, win_right=-1)
    # tile (qt 0, kt 0) of a 256 x 256 causal map is partial; compare it with an all-ones mask
    rb = torch.full((2 * 128,), -1, dtype=torch.int64, device=DEV)
    cb = torch.empty_like(rb)
    bad = torch.zeros(1, dtype=torch.int32, device=DEV)
    lst = torch.tensor([0, 0], dtype=torch.int32, device=DEV)
    st = torch.cuda.current_stream().cuda_stream
    _lib.check(lib.mattn_tilemap_bits(ctypes.byref(ms), 256, 256, 1, 1, lst.data_ptr(), 1, 1, 0,
                                      rb.data_ptr(), cb.data_ptr(), bad.data_ptr(), st))
    assert int(bad.item()) == 1
    # written then verified: no mismatch
    bad.zero_()
    _lib.check(lib.mattn_tilemap_bits(ctypes.byref(ms), 256, 256, 1, 1, lst.data_ptr(), 1, 1, 1,
                                      rb.data_ptr(), cb.data_ptr(), bad.data_ptr(), st))
    _lib.check(lib.mattn_tilemap_bits(ctypes.byref(ms), 256, 256, 1, 1, lst.data_ptr(), 1, 1, 0,
                                      rb.data_ptr(), cb.data_ptr(), bad.data_ptr(), st))
    assert int(bad.item()) == 0
    tri = np.tril(np.ones((128, 128), bool))
    assert np.array_equal(bmap.unpack_tile(rb.cpu().numpy().view(np.uint64).reshape(2, 128)), tri)
    assert np.array_equal(bmap.unpack_tile(cb.cpu().numpy().view(np.uint64).reshape(2, 128)), tri.T)
