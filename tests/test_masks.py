"""Closed-form masks (jaxmodules_amd.masks) on the CPU: each family evaluates
like the plain mask function it stands for, both elementwise (scalars, the
reference's calling convention) and through the host tracer, and bad
arguments raise before anything reaches the GPU."""
import ctypes
import os

import numpy as np
import pytest

from jaxmodules_amd import _lib
from jaxmodules_amd import blockmap as bmap
from jaxmodules_amd import masks


def assert_same_map(a, b):
    for f in ("map_b", "map_h", "pairs", "n_full", "n_partial"):
        assert getattr(a, f) == getattr(b, f), f
    for f in ("row_ptr", "row_ent", "col_ptr", "col_ent", "col_row", "row_bits", "col_bits",
              "q_order", "kv_order", "kv_desc"):
        assert np.array_equal(getattr(a, f), getattr(b, f)), f


def traced(shape_q, shape_k, **kw):
    return bmap.trace(bmap.make_plan(shape_q, shape_k, shape_k, **kw))


DOC = np.repeat(np.arange(7), [100, 37, 300, 5, 200, 158, 200])          # 1000 positions


def test_scalar_calls_follow_the_definitions():
    m = masks.intersect(masks.causal(), masks.window(3, 0), masks.documents(DOC))
    for q, k in [(5, 5), (5, 2), (5, 1), (4, 6), (99, 99), (100, 99), (120, 118)]:
        want = (q >= k) and (q - k <= 3) and DOC[q] == DOC[k]
        assert bool(m(0, 0, q, k)) == want, (q, k)
    w = masks.window(None, 2)
    assert bool(w(0, 0, 0, 2)) and not bool(w(0, 0, 0, 3)) and bool(w(0, 0, 900, 0))
    r = masks.intersect(masks.same_residue(5), masks.causal())
    for q, k in [(7, 2), (7, 7), (2, 7), (7, 3), (1000, 0), (1001, 1), (1001, 0)]:
        assert bool(r(0, 0, q, k)) == ((k % 5 == q % 5) and k <= q), (q, k)


def test_same_residue_is_the_benchmark_mask():
    """same_residue(P) & causal is check_attn.py:9-32's get_block_causal_mask
    (k <= q and k % P == q % P), written out here on a grid."""
    P, N = 16, 200
    q, k = np.arange(N)[:, None], np.arange(N)[None, :]
    want = (k <= q) & (k % P == q % P)
    got = masks.intersect(masks.same_residue(P), masks.causal())(0, 0, q, k)
    assert np.array_equal(np.broadcast_to(got, want.shape), want)


@pytest.mark.parametrize("case", ["causal_window", "docs", "docs_batch", "table", "cross", "residue",
                                  "residue_small", "residue_docs"])
def test_host_trace_equals_lambda(case):
    rng = np.random.default_rng(1)
    if case == "causal_window":
        sq = sk = (1, 1000, 2, 16)
        mf = masks.intersect(masks.causal(), masks.window(130, 0))
        lam = lambda b, h, q, k: (q >= k) & (q - k <= 130)                # noqa: E731
        kw = dict(block_size=50)
    elif case == "docs":
        sq = sk = (2, 1000, 2, 16)
        mf = masks.intersect(masks.documents(DOC), masks.causal())
        lam = lambda b, h, q, k: (DOC[q] == DOC[k]) & (q >= k)            # noqa: E731
        kw = dict(block_size=100)
    elif case == "docs_batch":
        sq = sk = (2, 1000, 2, 16)
        d2 = np.stack([DOC, DOC[::-1].copy()])
        mf = masks.documents(d2)
        lam = lambda b, h, q, k: d2[b, q] == d2[b, k]                      # noqa: E731
        kw = dict(block_size=100)
    elif case == "table":
        sq = sk = (1, 1000, 3, 16)
        t = rng.integers(0, 3, size=(3, 8, 8)).astype(np.uint8)
        mf = masks.intersect(masks.tile_table(t), masks.causal())
        lam = lambda b, h, q, k: (t[h, q // 128, k // 128] == 1) | (       # noqa: E731
            (t[h, q // 128, k // 128] == 2) & (q >= k))
        kw = dict(block_size=100)
    elif case == "residue":
        sq = sk = (1, 1000, 2, 16)
        mf = masks.intersect(masks.same_residue(160), masks.causal())
        lam = lambda b, h, q, k: ((q - k) % 160 == 0) & (q >= k)          # noqa: E731
        kw = dict(block_size=100)
    elif case == "residue_small":
        sq, sk = (1, 300, 2, 16), (1, 700, 2, 16)
        mf = masks.same_residue(7)
        lam = lambda b, h, q, k: k % 7 == q % 7                             # noqa: E731
        kw = dict(block_size=100)
    elif case == "residue_docs":
        sq = sk = (2, 1000, 2, 16)
        mf = masks.intersect(masks.same_residue(3), masks.documents(DOC), masks.window(200, 0))
        lam = lambda b, h, q, k: ((q - k) % 3 == 0) & (DOC[q] == DOC[k]) & (q - k <= 200) & (k <= q)  # noqa: E731
        kw = dict(block_size=100)
    else:
        sq, sk = (1, 300, 2, 16), (1, 700, 2, 16)
        dq, dk = np.arange(300) // 30, np.arange(700) // 70
        mf = masks.documents(dq, dk)
        lam = lambda b, h, q, k: dq[q] == dk[k]                            # noqa: E731
        kw = dict(block_size=100)
    assert_same_map(traced(sq, sk, mask_fn=mf, **kw), traced(sq, sk, mask_fn=lam, **kw))


def test_map_dims():
    assert masks.spec_of(masks.causal()).map_dims(4, 8) == (1, 1)
    assert masks.spec_of(masks.documents(np.zeros((4, 10), int))).map_dims(4, 8) == (4, 1)
    assert masks.spec_of(masks.documents(np.zeros(10, int))).map_dims(4, 8) == (1, 1)
    assert masks.spec_of(masks.tile_table(np.zeros((8, 1, 1), np.uint8))).map_dims(4, 8) == (1, 8)
    assert masks.spec_of(masks.tile_table(np.zeros((4, 1, 1, 1), np.uint8))).map_dims(4, 8) == (4, 1)


def test_intersect_rules():
    s = masks.spec_of(masks.intersect(masks.window(10, 5), masks.window(20, 2), masks.causal()))
    assert (s.win_left, s.win_right, s.causal) == (10, 2, True)
    with pytest.raises(ValueError):
        masks.intersect(masks.documents(DOC), masks.documents(DOC))
    with pytest.raises(ValueError):
        masks.intersect(masks.causal(), lambda b, h, q, k: q >= k)
    with pytest.raises(ValueError):
        masks.intersect()
    # two residue classes: the least common multiple
    assert masks.spec_of(masks.intersect(masks.same_residue(4), masks.same_residue(6))).period == 12


def test_argument_errors():
    with pytest.raises(ValueError):
        masks.window(-1, 0)
    with pytest.raises(ValueError):
        masks.documents(np.zeros((2, 3, 4), int))
    with pytest.raises(ValueError):
        masks.documents(np.zeros(10, np.float32))
    with pytest.raises(ValueError):
        masks.tile_table(np.full((2, 2), 3))
    for bad in (0, -3, 2.5, 2**31):
        with pytest.raises(ValueError):
            masks.same_residue(bad)
    spec = masks.spec_of(masks.documents(np.zeros(100, int)))
    with pytest.raises(ValueError):
        spec.check(1, 1, 99, 100)                       # ids of the wrong length
    spec = masks.spec_of(masks.tile_table(np.zeros((2, 2), np.uint8)))
    with pytest.raises(ValueError):
        spec.check(1, 1, 1000, 1000)                    # 8 x 8 tiles needed
    spec.check(1, 1, 256, 129)
    spec = masks.spec_of(masks.tile_table(np.zeros((3, 2, 2), np.uint8)))
    with pytest.raises(ValueError):
        spec.check(1, 4, 256, 256)                      # 3 head tables for 4 heads


def test_arrays_are_copied_and_frozen():
    d = DOC.copy()
    m = masks.documents(d)
    d[:] = 0
    s = masks.spec_of(m)
    assert s.doc_q.max() == 6
    with pytest.raises(ValueError):
        s.doc_q[0, 0] = 5


def test_device_trace_needs_closed_form():
    plan = bmap.make_plan((1, 64, 1, 16), (1, 64, 1, 16), (1, 64, 1, 16),
                          mask_fn=lambda b, h, q, k: q >= k)
    with pytest.raises(ValueError):
        bmap.device_trace(plan, "cuda:0")


@pytest.fixture(scope="module")
def lib():
    if not os.path.exists(_lib.LIB_PATH):
        pytest.skip("libmattn.so not built")
    return _lib.load()


def _spec(**kw):
    s = _lib.MattnMaskspec(causal=1, win_left=-1, win_right=-1)
    for k, v in kw.items():
        setattr(s, k, v)
    return s


def test_maskspec_validate_codes(lib):
    v = lambda s, Lq=1000, Lk=1000, mb=1, mh=1: lib.mattn_maskspec_validate(  # noqa: E731
        ctypes.byref(s), Lq, Lk, mb, mh)
    assert v(_spec()) == 0
    assert lib.mattn_maskspec_validate(None, 10, 10, 1, 1) == -1
    assert v(_spec(causal=2)) == -2
    assert v(_spec(), Lq=0) == -2
    assert v(_spec(win_left=-2)) == -2
    assert v(_spec(doc_b=1)) == -1                                  # ids missing
    assert v(_spec(doc_b=1, doc_q=8, doc_k=8)) == 0
    assert v(_spec(doc_b=3, doc_q=8, doc_k=8), mb=2) == -2          # neither 1 nor map_b
    assert v(_spec(doc_b=2, doc_q=8, doc_k=8), mb=2) == 0
    assert v(_spec(tab_b=1, tab_h=1)) == -1                         # table missing
    assert v(_spec(tab_b=1, tab_h=3, tiles=8), mh=4) == -2
    assert v(_spec(tab_b=1, tab_h=4, tiles=8), mh=4) == 0
    assert v(_spec(blk_size=128, blk_left=0, blk_right=0, blk_nk=8)) == -2
    assert v(_spec(blk_size=128, blk_left=4, blk_right=1, blk_nk=4)) == -2
    assert v(_spec(blk_size=128, blk_left=3, blk_right=1, blk_nk=4)) == 0
    assert v(_spec(), Lq=2**30, Lk=2**30) == -8                     # tile index beyond int32
    assert v(_spec(res_period=-1)) == -2
    assert v(_spec(res_period=2048)) == 0


def test_tilemap_entry_points_reject_before_launch(lib):
    s = _spec()
    assert lib.mattn_tilemap_classify(ctypes.byref(s), 100, 100, 1, 1, None, None, None, None) == -1
    assert lib.mattn_tilemap_bits(ctypes.byref(s), 100, 100, 1, 1, None, 1, 1, 1, None, None, None,
                                  None) == -1
    assert lib.mattn_tilemap_bits(ctypes.byref(s), 100, 100, 1, 1, None, -1, 1, 1, None, None, None,
                                  None) == -2
    assert lib.mattn_tilemap_bits(ctypes.byref(s), 100, 100, 1, 1, None, 0, 0, 1, None, None, None,
                                  None) == 0                          # nothing to do


def test_residue_view_is_the_class_major_permutation():
    """check_attn's mask k % P == q % P as P problems of length L / P:
    residue_view puts position s P + r at [r, s] without a copy, and
    residue_unview undoes it."""
    import torch

    from jaxmodules_amd import attention as A

    L, P, H, d = 48, 8, 3, 16
    x = torch.arange(L * H * d, dtype=torch.float32).reshape(1, L, H, d)
    v = A.residue_view(x, P)
    assert v.shape == (P, L // P, H, d) and v.data_ptr() == x.data_ptr()
    for r in range(P):
        for s in range(L // P):
            assert torch.equal(v[r, s], x[0, s * P + r])
    assert torch.equal(A.residue_unview(v), x)
    # within class r the mask (q - k) % P == 0 & k <= q is causal in the step index
    q, k = np.arange(L)[:, None], np.arange(L)[None, :]
    m = ((q - k) % P == 0) & (k <= q)
    for r in range(P):
        idx = np.arange(r, L, P)
        assert np.array_equal(m[np.ix_(idx, idx)], np.tril(np.ones((L // P, L // P), bool)))
        assert m[idx].sum() == m[np.ix_(idx, idx)].sum()      # no allowed key outside the class


@pytest.mark.parametrize("L,P", [(131072, 2048), (512, 16), (48, 8), (96, 12), (1024, 4), (640, 10)])
@pytest.mark.parametrize("causal", [True, False])
def test_residue_problem_packs_classes_without_changing_the_mask(L, P, causal):
    """residue_problem's rewrite of k % P == q % P (& k <= q): c classes per
    problem (the largest power of two dividing P with c L / P <= 128), and on
    every problem of the [P / c, c L / P] view the inner mask equals the
    original mask between the positions it stands for, while no allowed key
    lies outside the problem (brute force over the original L x L mask, or over
    the rows of a few problems at the largest size)."""
    from jaxmodules_amd import attention as A

    Pv, inner = A.residue_problem(L, P, causal)
    c = P // Pv
    assert Pv * c == P and c & (c - 1) == 0 and (c == 1 or c * (L // P) <= 128)
    assert P % (2 * c) or 2 * c * (L // P) > 128           # the largest such c
    n = L // Pv
    t = np.arange(n)
    if c == 1:
        assert inner == dict(is_causal=causal)
        im = np.tril(np.ones((n, n), bool)) if causal else np.ones((n, n), bool)
    else:
        spec = masks.spec_of(inner["mask_fn"])
        assert spec.period == c and spec.causal == causal and "is_causal" not in inner
        im = inner["mask_fn"](0, 0, t[:, None], t[None, :])
    for r in (range(Pv) if L <= 4096 else (0, 1, Pv // 2, Pv - 1)):
        pos = t * Pv + r
        q, k = pos[:, None], np.arange(L)[None, :]
        m = ((q - k) % P == 0) & ((k <= q) if causal else True)
        assert np.array_equal(m[:, pos], im)
        assert m.sum() == im.sum()                          # no allowed key outside the problem


def test_residue_rewrite_applies_only_to_plain_residue_masks():
    import torch

    from jaxmodules_amd import attention as A

    q = torch.zeros(1, 64, 2, 16)
    args = dict(kernel_fn=A.default_kernel, block_size=None, window_size=None, out_dtype=None, precision=None)
    for mf in (masks.intersect(masks.same_residue(8), masks.window(10, 0)), masks.causal(),
               masks.intersect(masks.same_residue(8), masks.documents(np.zeros(64, int)))):
        assert A._residue_rewrite(q, q, q, False, mask_fn=mf, **args) is None
    mf = masks.same_residue(7)                       # L % P != 0
    assert A._residue_rewrite(q, q, q, False, mask_fn=mf, **args) is None
    mf = masks.same_residue(8)
    assert A._residue_rewrite(torch.zeros(2, 64, 2, 16), torch.zeros(2, 64, 2, 16), torch.zeros(2, 64, 2, 16),
                              False, mask_fn=mf, **args) is None    # B > 1
    assert A._residue_rewrite(q, q, q, False, mask_fn=mf, kernel_fn=A.default_kernel, block_size=None,
                              window_size=(8, 0), out_dtype=None, precision=None) is None
