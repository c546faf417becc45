"""CPU oracle for the reference's ``block_mask.py`` -- TEST INFRASTRUCTURE ONLY.

Only ``tests/`` (and ``__graft_entry__.smoke()`` / ``bench.py``'s baseline leg)
may import this module.  It restates, with plain Python loops over numpy arrays,
the reference's tile classification and sparse-list construction:

* ``get_partial_block``            -- block_mask.py:381-408
* ``classify``                     -- create_block_mask, block_mask.py:454-498
  (partial = any XOR all, full = all)
* ``sparse_lists``                 -- get_sparse_kv_data_from_blocks, :411-432
  (num = row sum, indices = stable argsort of -blocks)
* ``create_block_mask``            -- :454-498 + from_blocks :227-275
* ``dense_from_lists``             -- get_dense_from_kv_blocks, :501-536
* ``materialize``                  -- BlockMask.materialize_mask, :68-129
* ``infer_kv_len``                 -- from_kv_blocks with seq_lengths=None, :303-339

Pinned in tests/test_oracle.py against the literal fixtures of the reference's
``tests/test_block_mask.py`` and against torch's own ``create_block_mask``.
"""
from __future__ import annotations

import numpy as np


def get_partial_block(mask_mod, b, h, qi, ki, QBS, KBS):
    out = np.zeros((QBS, KBS), dtype=bool)
    for r in range(QBS):
        for c in range(KBS):
            out[r, c] = bool(mask_mod(b, h, qi * QBS + r, ki * KBS + c))
    return out


def classify(mask_mod, B, H, Q_LEN, KV_LEN, QBS, KBS):
    """Returns (partial, full) int32 arrays [B, H, nq, nk]; partial excludes full."""
    nq, nk = Q_LEN // QBS, KV_LEN // KBS
    partial = np.zeros((B, H, nq, nk), np.int32)
    full = np.zeros((B, H, nq, nk), np.int32)
    for b in range(B):
        for h in range(H):
            for i in range(nq):
                for j in range(nk):
                    blk = get_partial_block(mask_mod, b, h, i, j, QBS, KBS)
                    a, e = blk.any(), blk.all()
                    partial[b, h, i, j] = int(a ^ e)
                    full[b, h, i, j] = int(e)
    partial = np.where(full != 0, 0, partial)
    return partial, full


def sparse_lists(blocks):
    """(num [.., rows], indices [.., rows, cols]) -- indices are the selected
    columns in ascending order followed by the unselected ones in ascending order."""
    blocks = np.asarray(blocks).astype(np.int32)
    if blocks.ndim == 2:
        blocks = blocks[None, None]
    num = blocks.sum(axis=-1).astype(np.int32)
    idx = np.zeros(blocks.shape, np.int32)
    for pos in np.ndindex(*blocks.shape[:-1]):
        row = blocks[pos]
        sel = [c for c in range(row.shape[0]) if row[c] != 0]
        rest = [c for c in range(row.shape[0]) if row[c] == 0]
        idx[pos] = np.array(sel + rest, np.int32)
    return num, idx


def create_block_mask(mask_mod, B, H, Q_LEN, KV_LEN, BLOCK_SIZE):
    QBS, KBS = (BLOCK_SIZE, BLOCK_SIZE) if isinstance(BLOCK_SIZE, int) else BLOCK_SIZE
    partial, full = classify(mask_mod, B, H, Q_LEN, KV_LEN, QBS, KBS)
    kv_num, kv_idx = sparse_lists(partial)
    q_num, q_idx = sparse_lists(partial.transpose(0, 1, 3, 2))
    fkv_num, fkv_idx = sparse_lists(full)
    fq_num, fq_idx = sparse_lists(full.transpose(0, 1, 3, 2))
    return dict(B=B, H=H, Q_LEN=(Q_LEN // QBS) * QBS, KV_LEN=(KV_LEN // KBS) * KBS,
                Q_BLOCK_SIZE=QBS, KV_BLOCK_SIZE=KBS,
                kv_num_blocks=kv_num, kv_indices=kv_idx,
                q_num_blocks=q_num, q_indices=q_idx,
                full_kv_num_blocks=fkv_num, full_kv_indices=fkv_idx,
                full_q_num_blocks=fq_num, full_q_indices=fq_idx, mask_mod=mask_mod)


def dense_from_lists(B, H, rows, cols, num, idx):
    out = np.zeros((B, H, rows, cols), bool)
    for b in range(B):
        for h in range(H):
            for i in range(rows):
                for j in range(int(num[b, h, i])):
                    out[b, h, i, int(idx[b, h, i, j])] = True
    return out


def materialize(bm):
    """Dense int32 [B, H, Q_LEN, KV_LEN]: partial tiles filled from mask_mod,
    full tiles set to one (BlockMask.materialize_mask)."""
    B, H = bm["B"], bm["H"]
    QBS, KBS = bm["Q_BLOCK_SIZE"], bm["KV_BLOCK_SIZE"]
    out = np.zeros((B, H, bm["Q_LEN"], bm["KV_LEN"]), np.int32)
    nq = bm["kv_num_blocks"].shape[-1]
    for b in range(B):
        for h in range(H):
            for i in range(nq):
                for s in range(int(bm["kv_num_blocks"][b, h, i])):
                    j = int(bm["kv_indices"][b, h, i, s])
                    if j * KBS >= bm["KV_LEN"]:
                        continue  # an out-of-range scatter is dropped (jax .at[].set)
                    out[b, h, i * QBS:(i + 1) * QBS, j * KBS:(j + 1) * KBS] = get_partial_block(
                        bm["mask_mod"], b, h, i, j, QBS, KBS)
                # jax clamps an out-of-range gather index (the fixture at
                # test_block_mask.py:87-88 lists fewer full rows than query blocks)
                fn, fi = bm["full_kv_num_blocks"], bm["full_kv_indices"]
                ic = min(i, fn.shape[-1] - 1)
                for s in range(int(fn[b, h, ic])):
                    j = int(fi[b, h, min(ic, fi.shape[2] - 1), s])
                    if j * KBS >= bm["KV_LEN"]:
                        continue
                    out[b, h, i * QBS:(i + 1) * QBS, j * KBS:(j + 1) * KBS] = 1
    return out


def infer_kv_len(kv_num, kv_idx, fkv_num, fkv_idx, KBS):
    """KV_LEN = (max listed index over partial and full lists + 1) * KV block size."""
    best = -1
    for num, idx in ((kv_num, kv_idx), (fkv_num, fkv_idx)):
        num = np.asarray(num)
        idx = np.asarray(idx)
        for pos in np.ndindex(*num.shape):
            for s in range(int(num[pos])):
                best = max(best, int(idx[pos + (s,)]))
    return (best + 1) * KBS
