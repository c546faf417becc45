"""The host tile-map tracer against the oracle (CPU only).

The traced map, expanded back to a dense mask, must equal the oracle's
effective mask (mask_fn AND window AND unpadded range) exactly; the pair count
(the FLOP basis of the metric) must equal the oracle's count and the BASELINE
closed forms; the CSR row and column lists, the de-duplicated bitmasks and the
launch orders must be mutually consistent.
"""
import numpy as np
import pytest

from jaxmodules_amd import blockmap as bm
from oracle import attention_oracle as ao

CASES = {
    "causal_gqa_pad": ((2, 300, 4, 64), (2, 300, 2, 64), dict(is_causal=True, block_size=32)),
    "three_arg_no_bs": ((1, 256, 2, 64), (1, 512, 2, 64),
                        dict(mask_fn=lambda h, q, k: (q - k) % 3 != 1)),
    "window_mask": ((2, 640, 2, 64), (2, 640, 2, 64),
                    dict(mask_fn=lambda b, h, q, k: (q >= k) & (q - k <= 200), block_size=128,
                         window_size=(200, 0))),
    "window_only": ((1, 512, 2, 64), (1, 512, 2, 64), dict(block_size=64, window_size=(64, 64))),
    "batch_head_docs": ((2, 333, 3, 64), (2, 333, 3, 64),
                        dict(mask_fn=lambda b, h, q, k: (q // (50 + b * 7 + h)) == (k // (50 + b * 7 + h)),
                             block_size=10)),
    "ragged_tiny": ((1, 10, 4, 64), (1, 13, 4, 64),
                    dict(mask_fn=lambda h, q, k: abs(q - k) <= 2, block_size=4)),
    "empty_rows": ((1, 256, 2, 64), (1, 256, 2, 64),
                   dict(mask_fn=lambda b, h, q, k: (q > 100) & (k <= q), block_size=128)),
    "nothing_allowed": ((1, 200, 2, 64), (1, 200, 2, 64),
                        dict(mask_fn=lambda b, h, q, k: q < 0, block_size=100)),
}


@pytest.mark.parametrize("name", sorted(CASES))
def test_trace_equals_oracle_mask(name):
    qs, ks, kw = CASES[name]
    plan = bm.make_plan(qs, ks, ks, **kw)
    tm = bm.trace(plan)
    ref = ao.effective_mask(ao.canonical_plan(qs, ks, ks, **kw))
    assert np.array_equal(np.broadcast_to(tm.dense(), ref.shape), ref)
    assert tm.pairs == int(ref.sum())
    check_consistency(tm, plan)


def check_consistency(tm, plan):
    nmap = tm.map_b * tm.map_h
    # row CSR: key tiles ascending within each row, ids in range
    for r in range(nmap * tm.nqt):
        ent = tm.row_ent[tm.row_ptr[r]:tm.row_ptr[r + 1]]
        assert np.all(np.diff(ent[:, 0]) > 0)
        assert np.all((ent[:, 1] >= -1) & (ent[:, 1] < tm.n_masks))
    # column CSR lists exactly the transposed entries
    rows = np.repeat(np.arange(nmap * tm.nqt), np.diff(tm.row_ptr))
    fwd = {(r // tm.nqt, r % tm.nqt, int(kt), int(m)) for r, (kt, m) in zip(rows, tm.row_ent)}
    cols = np.repeat(np.arange(nmap * tm.nkt), np.diff(tm.col_ptr))
    bwd = {(c // tm.nkt, int(qt), c % tm.nkt, int(m)) for c, (qt, m) in zip(cols, tm.col_ent)}
    assert fwd == bwd
    # col_row names, for every column entry, the row entry of the same tile (a permutation)
    assert tm.col_row.dtype == np.int32 and tm.col_row.shape == (tm.nnz,)
    assert np.array_equal(np.sort(tm.col_row), np.arange(tm.nnz))
    r_of = rows[tm.col_row]
    assert np.array_equal(r_of // tm.nqt, cols // tm.nkt)                 # same map slab
    assert np.array_equal(r_of % tm.nqt, tm.col_ent[:, 0])                # same query tile
    assert np.array_equal(tm.row_ent[tm.col_row, 0], cols % tm.nkt)       # same key tile
    assert np.array_equal(tm.row_ent[tm.col_row, 1], tm.col_ent[:, 1])   # same mask
    # kv_desc: per launch slot, the column's first entry, recomputed by plain loops
    G = plan.Hq // plan.Hkv
    assert tm.kv_desc.dtype == np.int32 and tm.kv_desc.shape == (len(tm.kv_order), 8)
    for slot, item in enumerate(tm.kv_order):
        d = tm.kv_desc[slot]
        if item < 0:
            assert d[0] == -1 and not d[1:].any()
            continue
        kt, bhk = item % tm.nkt, item // tm.nkt
        hk, b = bhk % plan.Hkv, bhk // plan.Hkv
        ranges = []
        for g in range(G):
            mc = ((b % tm.map_b) * tm.map_h + (hk * G + g) % tm.map_h) * tm.nkt + kt
            ranges.append((g, tm.col_ptr[mc], tm.col_ptr[mc + 1]))
        tot = 2 * sum(e1 - e0 for _, e0, e1 in ranges)
        assert d[0] == item and d[4] == tot
        nonempty = [r for r in ranges if r[2] > r[1]]
        if not nonempty:
            assert not d[1:].any()
            continue
        g, e0, e1 = nonempty[0]
        assert tuple(d[1:4]) == (g, e0, e1)
        assert tuple(d[5:8]) == (tm.col_ent[e0, 0], tm.col_ent[e0, 1], tm.col_row[e0])
    # masks are distinct and the column bits are the transposed row bits
    seen = set()
    for m in range(tm.n_masks):
        rbits = bm.unpack_tile(tm.row_bits[m])
        cbits = bm.unpack_tile(tm.col_bits[m])
        assert np.array_equal(rbits.T, cbits)
        assert 0 < rbits.sum() < 128 * 128
        assert rbits.tobytes() not in seen
        seen.add(rbits.tobytes())
    # launch orders cover every work item exactly once
    q = tm.q_order[tm.q_order >= 0]
    assert sorted(q.tolist()) == list(range(plan.B * plan.Hq * tm.nqt))
    kv = tm.kv_order[tm.kv_order >= 0]
    assert sorted(kv.tolist()) == list(range(plan.B * plan.Hkv * tm.nkt))
    assert tm.q_order.size % bm.NUM_XCD == 0


def test_causal_pairs_closed_form_cfg2():
    """BASELINE cfg2: causal B=4 L=4096 H=32 -> 1.0740e9 pairs, one shared diagonal mask."""
    plan = bm.make_plan((4, 4096, 32, 128), (4, 4096, 32, 128), (4, 4096, 32, 128), is_causal=True,
                        block_size=128)
    tm = bm.trace(plan)
    assert tm.pairs == 4 * 32 * 4096 * 4097 // 2 == 1074003968
    assert (tm.map_b, tm.map_h) == (1, 1)
    assert tm.n_masks == 1 and tm.n_partial == 32 and tm.n_full == 32 * 31 // 2


def test_window_cfg3_tile_pattern():
    """cfg3: (q>=k)&(q-k<=512), window (512,0), block 128: each query tile sees
    3 full + 2 partial key tiles away from the start; 2.6476e8 pairs."""
    mask = lambda b, h, q, k: (q >= k) & (q - k <= 512)
    plan = bm.make_plan((2, 16384, 16, 128), (2, 16384, 16, 128), (2, 16384, 16, 128), mask_fn=mask,
                        window_size=(512, 0), block_size=128)
    tm = bm.trace(plan)
    per_row = 513 * 16384 - 512 * 513 // 2
    assert tm.pairs == 2 * 16 * per_row
    st = tm.states()[0, 0]
    for i in range(5, 128):
        assert (st[i] == 1).sum() == 3 and (st[i] == 2).sum() == 2


def test_head_dependence_probe():
    B, H = 3, 4
    assert bm._probe_dependence(lambda b, h, q, k: q >= k, B, H, 8, 8) == (1, 1)
    assert bm._probe_dependence(lambda b, h, q, k: (q + h) >= k, B, H, 8, 8) == (1, H)
    assert bm._probe_dependence(lambda b, h, q, k: (q + b) >= k, B, H, 8, 8) == (B, 1)
    assert bm._probe_dependence(lambda b, h, q, k: True, B, H, 8, 8) == (1, 1)


def test_lpt_xcd_order():
    w = np.array([5, 1, 9, 3, 7, 2, 8, 6, 4, 10, 11, 12, 0, 13, 14, 15])
    g = np.arange(16) // 2          # 8 groups of two items
    o = bm._lpt_xcd_order(w, g)
    assert sorted(o[o >= 0].tolist()) == list(range(16))
    slots = o.reshape(-1, bm.NUM_XCD)
    for x in range(bm.NUM_XCD):      # one XCD's items: one group, heaviest first
        col = [i for i in slots[:, x] if i >= 0]
        assert len({int(g[i]) for i in col}) <= 1
        assert list(w[col]) == sorted(w[col], reverse=True)


@pytest.mark.parametrize("ngroups", [1, 2, 3])
def test_lpt_xcd_order_few_groups(ngroups):
    """Fewer groups than XCDs: each group's items go round-robin (by their
    index within the group) over NUM_XCD // ngroups XCDs of their own, so that
    every die has work; heaviest first on each XCD."""
    per = 40
    g = np.repeat(np.arange(ngroups), per)
    w = np.tile(np.arange(per), ngroups) + 1       # causal-like: later items heavier
    o = bm._lpt_xcd_order(w, g)
    assert sorted(o[o >= 0].tolist()) == list(range(g.size))
    slots = o.reshape(-1, bm.NUM_XCD)
    spread = bm.NUM_XCD // ngroups
    used = [x for x in range(bm.NUM_XCD) if (slots[:, x] >= 0).any()]
    assert len(used) == ngroups * spread
    for x in used:
        col = [int(i) for i in slots[:, x] if i >= 0]
        assert len({int(g[i]) for i in col}) == 1               # one group per XCD
        assert len(col) == per // spread or len(col) == per // spread + 1
        assert list(w[col]) == sorted(w[col], reverse=True)


def test_lpt_xcd_order_blocks_of_groups():
    """An XCD with more than HEADS_AT_ONCE groups takes them block by block,
    heaviest first inside a block."""
    rng = np.random.default_rng(3)
    ng, per = 8 * 3 * bm.HEADS_AT_ONCE, 5          # three blocks per XCD
    g = np.repeat(np.arange(ng), per)
    w = rng.integers(1, 100, size=g.size)
    o = bm._lpt_xcd_order(w, g)
    assert sorted(o[o >= 0].tolist()) == list(range(g.size))
    slots = o.reshape(-1, bm.NUM_XCD)
    for x in range(bm.NUM_XCD):
        col = [int(i) for i in slots[:, x] if i >= 0]
        assert all(g[i] % bm.NUM_XCD == x for i in col)
        blocks = [(g[i] // bm.NUM_XCD) // bm.HEADS_AT_ONCE for i in col]
        assert blocks == sorted(blocks)
        for blk in set(blocks):
            ws = [w[i] for i, b_ in zip(col, blocks) if b_ == blk]
            assert ws == sorted(ws, reverse=True)


def test_reference_exceptions():
    with pytest.raises(ValueError):
        bm.make_plan((8, 4, 16), (8, 4, 16), (8, 4, 16), is_causal=True, mask_fn=lambda h, a, b: True)
    with pytest.raises(ValueError):
        bm.make_plan((8, 16), (8, 16), (8, 16))
    with pytest.raises(AssertionError):
        bm.make_plan((8, 4, 16), (8, 4, 17), (8, 4, 16))
    with pytest.raises(AssertionError):
        bm.make_plan((8, 6, 16), (8, 4, 16), (8, 4, 16))
    with pytest.raises(TypeError):
        bm.make_plan((8, 1, 4), (8, 1, 4), (8, 1, 4), window_size=(1, 0))
