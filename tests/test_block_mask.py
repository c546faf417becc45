"""BlockMask (CPU): the reference tests' literal fixtures
(/root/reference/tests/test_block_mask.py), agreement with torch's
``create_block_mask`` (an independent implementation of the same
classification, which the reference's own flex_attention tests compare
against), brute force on tiny masks, and the hand-over to the kernels' tile map.
"""
import numpy as np
import pytest

from jaxmodules_amd import block_mask as bmk
from jaxmodules_amd.block_mask import (BlockMask, array_from_coords, create_block_mask,
                                       get_dense_from_kv_blocks, get_partial_block,
                                       get_sparse_kv_data_from_blocks,
                                       get_sparse_q_data_from_blocks, nested_fori_loop)

CAUSAL8 = np.tril(np.ones((8, 8), np.int32))


# --- the reference tests' fixtures ------------------------------------------


def test_block_mask_basic():
    """test_block_mask.py:15-51"""
    B, H, L, bs = 2, 2, 8, 4
    bm = create_block_mask(lambda b, h, q, k: q >= k, B, H, L, L, bs)
    assert (bm.B, bm.H, bm.Q_LEN, bm.KV_LEN, bm.Q_BLOCK_SIZE, bm.KV_BLOCK_SIZE) == (B, H, L, L, bs, bs)
    dense = bm.materialize_mask()
    assert dense.dtype == np.int32
    assert np.array_equal(dense, np.broadcast_to(CAUSAL8, (B, H, L, L)))


def test_block_mask_partial_blocks():
    """test_block_mask.py:54-72"""
    bm = create_block_mask(lambda b, h, q, k: (q + k) % 3 == 0, 1, 1, 8, 8, 4)
    q, k = np.meshgrid(np.arange(8), np.arange(8), indexing="ij")
    assert np.array_equal(bm.materialize_mask()[0, 0], ((q + k) % 3 == 0).astype(np.int32))


def test_block_mask_from_kv_blocks():
    """test_block_mask.py:75-113: index 4 of the last row lies past the 4 key
    blocks (dropped), and the full lists are shorter than the rows (clamped)."""
    L, bs = 8, 2
    bm = BlockMask.from_kv_blocks(
        kv_num_blocks=np.array([[[2, 2, 2, 2]]]),
        kv_indices=np.array([[[[0, 1], [1, 2], [2, 3], [3, 4]]]]),
        full_kv_num_blocks=np.array([[[0, 0]]]),
        full_kv_indices=np.array([[[[0, 0], [0, 0]]]]),
        BLOCK_SIZE=bs,
        mask_mod=lambda b, h, q, k: (k // bs >= q // bs) & (k // bs <= q // bs + 1),
        seq_lengths=(L, L))
    dense = bm.materialize_mask()
    q, k = np.meshgrid(np.arange(L), np.arange(L), indexing="ij")
    want = (k // bs >= q // bs) & (k // bs < q // bs + 2)
    assert np.array_equal(dense[0, 0], want.astype(np.int32))
    assert bm.q_num_blocks is None and bm.full_q_indices is None


def test_block_mask_from_kv_blocks_no_seq_len():
    """test_block_mask.py:116-169: Q_LEN = 3 rows x 2, KV_LEN = (max index 3 + 1) x 2."""
    bm = BlockMask.from_kv_blocks(
        kv_num_blocks=np.array([[[1, 2, 1]]]),
        kv_indices=np.array([[[[0, 3], [1, 2], [3, 3]]]]),
        full_kv_num_blocks=np.array([[[1, 0, 1]]]),
        full_kv_indices=np.array([[[[2, 0], [0, 0], [1, 0]]]]),
        BLOCK_SIZE=2,
        mask_mod=lambda b, h, q, k: (q + k) % 2 == 0)
    assert (bm.Q_LEN, bm.KV_LEN, bm.B, bm.H, bm.Q_BLOCK_SIZE, bm.KV_BLOCK_SIZE) == (6, 8, 1, 1, 2, 2)
    dense = bm.materialize_mask()
    assert dense.shape == (1, 1, 6, 8) and dense.min() >= 0 and dense.max() <= 1
    # brute force: listed partial tiles follow the parity rule, listed full tiles are ones
    q, k = np.meshgrid(np.arange(6), np.arange(8), indexing="ij")
    want = np.zeros((6, 8), bool)
    for qb, kbs in ((0, [0]), (1, [1, 2]), (2, [3])):
        for kb in kbs:
            s = (slice(2 * qb, 2 * qb + 2), slice(2 * kb, 2 * kb + 2))
            want[s] = ((q + k) % 2 == 0)[s]
    for qb, kb in ((0, 2), (2, 1)):
        want[2 * qb:2 * qb + 2, 2 * kb:2 * kb + 2] = True
    assert np.array_equal(dense[0, 0], want.astype(np.int32))


def test_get_partial_block():
    """test_block_mask.py:172-185"""
    blk = get_partial_block(lambda b, h, q, k: (q + k) % 2 == 0, 0, 0, 0, 0, 4, 4, 1, 1)
    assert np.array_equal(blk, np.array([[1, 0, 1, 0], [0, 1, 0, 1], [1, 0, 1, 0], [0, 1, 0, 1]]))
    blk = get_partial_block(lambda b, h, q, k: q >= k + 3, 0, 0, 1, 0, 2, 3, 1, 1)
    assert np.array_equal(blk, np.array([[False, False, False], [True, False, False]]))


def test_get_sparse_kv_data_from_blocks():
    """test_block_mask.py:188-222, including the [rows, cols] input."""
    rel = np.array([[True, False], [True, True]])
    for blocks in (np.array([[[[1, 0], [1, 1]]]]), np.array([[1, 0], [1, 1]])):
        num, idx = get_sparse_kv_data_from_blocks(blocks)
        assert num.dtype == np.int32 and idx.dtype == np.int32
        assert np.array_equal(num, [[[1, 2]]])
        assert np.array_equal(idx * rel, np.array([[[[0, 2], [0, 1]]]]) * rel)


def test_get_sparse_q_data_from_blocks():
    """test_block_mask.py:225-246"""
    num, idx = get_sparse_q_data_from_blocks(np.array([[[[1, 0], [1, 1]]]]))
    rel = np.array([[True, True], [True, False]])
    assert np.array_equal(num, [[[2, 1]]])
    assert np.array_equal(idx * rel, np.array([[[[0, 1], [1, 2]]]]) * rel)


def test_get_dense_from_kv_blocks():
    """test_block_mask.py:249-265"""
    dense = get_dense_from_kv_blocks(1, 1, 2, 2, np.array([[[1, 2]]]), np.array([[[[0, 0], [0, 1]]]]))
    assert dense.dtype == bool
    assert np.array_equal(dense, [[[[1, 0], [1, 1]]]])


def test_block_mask_causal_mask():
    """test_block_mask.py:268-301"""
    bm = BlockMask.causal_mask(2, 2, 8, 8, 4)
    assert (bm.B, bm.H, bm.Q_LEN, bm.KV_LEN, bm.Q_BLOCK_SIZE, bm.KV_BLOCK_SIZE) == (2, 2, 8, 8, 4, 4)
    assert np.array_equal(bm.materialize_mask(), np.broadcast_to(CAUSAL8, (2, 2, 8, 8)))
    assert np.array_equal(bm.to_dense()[0, 0], [[1, 0], [1, 1]])
    assert np.array_equal(bm.get_full_blocks()[0, 0], [[0, 0], [1, 0]])
    assert np.array_equal(bm.get_partial_blocks()[0, 0], [[1, 0], [0, 1]])


def test_block_mask_full_mask():
    """test_block_mask.py:304-323"""
    bm = BlockMask.full_mask(2, 2, 8, 8, 4)
    assert (bm.B, bm.H, bm.Q_LEN, bm.KV_LEN) == (2, 2, 8, 8)
    assert np.array_equal(bm.materialize_mask(), np.ones((2, 2, 8, 8), np.int32))
    assert bm.q_num_blocks is None          # from_kv_blocks without generate_q_blocks
    with pytest.raises(AttributeError):
        bm.to_dense()


def test_from_kv_blocks_rejects_low_rank_lists():
    """The reference's "... q -> 1 1 q" rearrange (block_mask.py:291-298) raises
    a RuntimeError (einops) for every input of fewer dimensions."""
    with pytest.raises(RuntimeError):
        BlockMask.from_kv_blocks(np.array([1, 1]), np.array([[[[0], [1]]]]), np.array([[[0, 0]]]),
                                 np.array([[[[0], [0]]]]), 2, lambda b, h, q, k: True)


# --- against torch's create_block_mask (CPU) ---------------------------------

MASKS = {
    "causal": lambda b, h, q, k: q >= k,
    "sliding": lambda b, h, q, k: abs(q - k) <= 5,
    "mod3": lambda b, h, q, k: (q + k) % 3 == 0,
    "head": lambda b, h, q, k: (q + 4 * h) >= k,
    "batch_doc": lambda b, h, q, k: (q // (6 + 5 * b)) == (k // (6 + 5 * b)),
    "nothing": lambda b, h, q, k: q < 0,
    "prefix": lambda b, h, q, k: (k < 8) | (q >= k),
}


@pytest.mark.parametrize("name", sorted(MASKS))
@pytest.mark.parametrize("shape", [(2, 3, 32, 32, 8), (1, 2, 24, 40, 8), (2, 2, 32, 16, (8, 4))])
def test_matches_torch_create_block_mask(name, shape):
    torch = pytest.importorskip("torch")
    from torch.nn.attention.flex_attention import create_block_mask as torch_cbm

    B, H, Q, KV, bs = shape
    fn = MASKS[name]
    ours = create_block_mask(fn, B, H, Q, KV, bs)
    theirs = torch_cbm(fn, B, H, Q, KV, device="cpu", BLOCK_SIZE=bs, _compile=False)
    nq, nk = Q // bmk.extract_block_size(bs)[0], KV // bmk.extract_block_size(bs)[1]
    for f in ("kv_num_blocks", "kv_indices", "full_kv_num_blocks", "full_kv_indices",
              "q_num_blocks", "q_indices", "full_q_num_blocks", "full_q_indices"):
        t = getattr(theirs, f).numpy()
        o = getattr(ours, f)
        o = np.broadcast_to(o, (t.shape[0], t.shape[1]) + o.shape[2:])
        assert o.dtype == np.int32, f
        assert np.array_equal(o[..., :t.shape[2], :], t) if o.ndim == 4 else np.array_equal(o, t), f
    # the dense mask is the mask_fn itself (every element lies in a listed tile)
    b, h, q, k = np.ix_(np.arange(B), np.arange(H), np.arange(Q), np.arange(KV))
    want = np.broadcast_to(np.asarray(fn(b, h, q, k), bool), (B, H, Q, KV))
    assert np.array_equal(ours.materialize_mask().astype(bool), want)
    assert nq * nk > 0


# --- brute force ---------------------------------------------------------------


def test_create_block_mask_brute_force():
    rng = np.random.default_rng(3)
    for _ in range(20):
        B, H = rng.integers(1, 3, size=2)
        bq, bk = rng.integers(1, 5, size=2)
        nq, nk = rng.integers(1, 5, size=2)
        tbl = rng.random((B, H, nq * bq, nk * bk)) < rng.choice([0.1, 0.5, 0.95])
        fn = lambda b, h, q, k: tbl[b, h, q, k]
        bm = create_block_mask(fn, B, H, nq * bq, nk * bk, (bq, bk))
        t = tbl.reshape(B, H, nq, bq, nk, bk)
        full = t.all(axis=(3, 5))
        part = t.any(axis=(3, 5)) & ~full
        assert np.array_equal(bm.get_full_blocks(), full)
        assert np.array_equal(bm.get_partial_blocks(), part)
        assert np.array_equal(bm.materialize_mask().astype(bool), tbl)
        # lists: first num entries are the marked columns ascending, then the rest ascending
        for bb in range(B):
            for hh in range(H):
                for i in range(nq):
                    row = part[bb, hh, i]
                    want = np.concatenate([np.nonzero(row)[0], np.nonzero(~row)[0]])
                    assert np.array_equal(bm.kv_indices[bb, hh, i], want)
                    assert bm.kv_num_blocks[bb, hh, i] == row.sum()
        # from_kv_blocks(generate_q_blocks) round-trips every list
        bm2 = BlockMask.from_kv_blocks(bm.kv_num_blocks, bm.kv_indices, bm.full_kv_num_blocks,
                                       bm.full_kv_indices, (bq, bk), fn,
                                       seq_lengths=(nq * bq, nk * bk), generate_q_blocks=True)
        for f in ("kv_num_blocks", "kv_indices", "q_num_blocks", "q_indices", "full_kv_num_blocks",
                  "full_kv_indices", "full_q_num_blocks", "full_q_indices"):
            assert np.array_equal(getattr(bm, f), getattr(bm2, f)), f


def test_grid_helpers():
    """vectorize.py:9-33 and the nested_fori_loop docstring examples (:203-226)."""
    a = array_from_coords((2, 3), lambda i, j: 10 * i + j)
    assert np.array_equal(a, [[0, 1, 2], [10, 11, 12]])
    assert np.array_equal(array_from_coords((2, 2), lambda i, j: 7), np.full((2, 2), 7))
    seen = nested_fori_loop((0, 0), (2, 3), lambda i, j, v: v + [(i, j)], [])
    assert seen == [(i, j) for i in range(2) for j in range(3)]
    seen = nested_fori_loop((0, lambda i: i), (2, lambda i: i + 3), lambda i, j, v: v + [(i, j)], [])
    assert seen == [(i, j) for i in range(2) for j in range(i, i + 3)]
    assert nested_fori_loop((0, 0, 0), (2, 2, lambda i, j: i + j), lambda i, j, k, v: v + 1, 0) == 4


# --- hand-over to the kernels ----------------------------------------------------


@pytest.mark.parametrize("bs", [16, 64, 128, 200, (64, 32)])
def test_tile_map_equals_materialized_mask(bs):
    """The kernels' tile map of a BlockMask expands to materialize_mask()."""
    Qb, KVb = bmk.extract_block_size(bs)
    L = 400 if bs == 200 else 384
    for name, fn in (("causal", MASKS["causal"]), ("head", MASKS["head"]),
                     ("batch_doc", MASKS["batch_doc"]), ("nothing", MASKS["nothing"])):
        bm = create_block_mask(fn, 2, 4, L, L, bs)
        tm = bm.tile_map(2, 4, 4)
        ref = bm.materialize_mask().astype(bool)
        assert np.array_equal(np.broadcast_to(tm.dense(), ref.shape), ref), name
        assert tm.pairs == int(ref.sum())
    bm = BlockMask.causal_mask(1, 1, L, L, bs)
    tm = bm.tile_map(3, 4, 2)
    assert (tm.map_b, tm.map_h) == (1, 1)
    assert np.array_equal(tm.dense()[0, 0], bm.materialize_mask()[0, 0].astype(bool))


def test_tile_map_gqa_uses_kv_head_for_elements():
    """flex_attention evaluates a partial tile's elements with the KV head index
    (attention.py:561-575) while the lists are read with the query head."""
    fn = lambda b, h, q, k: (q + 8 * h) >= k
    bm = create_block_mask(fn, 1, 4, 64, 64, 16)
    tm = bm.tile_map(1, 4, 2)
    dense = tm.dense()[0]
    lists = bm.to_dense()[0]                                  # tiles of query head hq
    for hq in range(4):
        q, k = np.meshgrid(np.arange(64), np.arange(64), indexing="ij")
        elem = (q + 8 * (hq // 2)) >= k
        full = np.kron(bm.get_full_blocks()[0, hq], np.ones((16, 16), bool))
        part = np.kron(bm.get_partial_blocks()[0, hq], np.ones((16, 16), bool))
        assert np.array_equal(dense[hq], full | (part & elem))
        assert lists[hq].any()


def test_tile_map_rejects_unrepresentable_lists():
    bm = BlockMask.causal_mask(1, 1, 8, 8, 4)
    with pytest.raises(ValueError):                      # B=2 mask, 3 batches
        BlockMask.causal_mask(2, 1, 8, 8, 4).tile_map(3, 1, 1)
    twice = BlockMask.from_kv_blocks(np.array([[[1, 1]]]), np.array([[[[0], [0]]]]),
                                     np.array([[[1, 0]]]), np.array([[[[0], [0]]]]), 4,
                                     lambda b, h, q, k: q >= k, seq_lengths=(8, 8))
    with pytest.raises(ValueError):
        twice.tile_map(1, 1, 1)
    outside = BlockMask.from_kv_blocks(np.array([[[1, 0]]]), np.array([[[[2], [0]]]]),
                                       np.array([[[0, 0]]]), np.array([[[[0], [0]]]]), 4,
                                       lambda b, h, q, k: q >= k, seq_lengths=(8, 8))
    with pytest.raises(ValueError):
        outside.tile_map(1, 1, 1)
    assert bm.tile_map(1, 1, 1).pairs == 36


def test_matches_loop_oracle():
    """The vectorised module against the loop-level restatement in
    oracle/block_mask_oracle.py (itself pinned in test_oracle.py)."""
    from oracle import block_mask_oracle as bo

    rng = np.random.default_rng(11)
    for bs, (B, H, Q, KV) in (((4, 4), (2, 3, 16, 24)), ((8, 2), (1, 2, 24, 16)), ((3, 5), (2, 1, 12, 20))):
        tbl = rng.random((B, H, Q, KV)) < 0.6
        fn = lambda b, h, q, k: tbl[b, h, q, k]
        ours = create_block_mask(fn, B, H, Q, KV, bs)
        ref = bo.create_block_mask(fn, B, H, Q, KV, bs)
        for f in ("kv_num_blocks", "kv_indices", "q_num_blocks", "q_indices", "full_kv_num_blocks",
                  "full_kv_indices", "full_q_num_blocks", "full_q_indices"):
            assert np.array_equal(getattr(ours, f), ref[f]), f
        assert (ours.Q_LEN, ours.KV_LEN) == (ref["Q_LEN"], ref["KV_LEN"])
        assert np.array_equal(ours.materialize_mask(), bo.materialize(ref))
    kv_num, kv_idx = np.array([[[1, 2, 1]]]), np.array([[[[0, 3], [1, 2], [3, 3]]]])
    fkv_num, fkv_idx = np.array([[[1, 0, 1]]]), np.array([[[[2, 0], [0, 0], [1, 0]]]])
    bm = BlockMask.from_kv_blocks(kv_num, kv_idx, fkv_num, fkv_idx, 2, lambda b, h, q, k: q >= k)
    assert bm.KV_LEN == bo.infer_kv_len(kv_num, kv_idx, fkv_num, fkv_idx, 2)
