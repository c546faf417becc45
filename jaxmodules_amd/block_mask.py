"""Block-sparse mask descriptor (the reference's ``block_mask.py``), host side.

``BlockMask`` classifies the (query block, key block) tiles of a mask into
*full* tiles (every element allowed), *partial* tiles (some allowed: the
element mask comes from ``mask_mod``) and empty tiles (absent), and stores the
two kinds as padded per-row index lists, plus the transposed per-column lists
(``/root/reference/jaxmodules/block_mask.py:17-42``).  The fields, their
dtypes (int32 counts and indices) and the list order (listed tiles first in
ascending index, then the unlisted ones ascending: a stable descending argsort,
block_mask.py:428-430) follow the reference, so a mask built by either side
means the same thing.

Host arrays are numpy.  ``mask_mod(b, h, q, k)`` is called with index arrays
that broadcast against each other, as ``mask_fn`` is for
``masked_attention_via_map``; the reference calls it with scalars under nested
``vmap`` (vectorize.py:9-33), so any elementwise function of the indices works
in both.  Where the reference indexes its arrays with computed indices, the
functions here reproduce what jax does with an index out of range: a read is
clamped to the nearest valid position, a write is dropped (negative indices
count from the end).

``BlockMask.tile_map`` hands a mask to the MI355X kernels: it re-tiles the
descriptor into the kernels' 128 x 128 tile map, with the element semantics of
the reference's ``flex_attention`` (attention.py:456-692).
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Callable, Optional, Tuple

import numpy as np

from . import blockmap as _bm

# elements evaluated per vectorised mask_mod call
_CHUNK = 1 << 24


def extract_block_size(BLOCK_SIZE) -> Tuple[int, int]:
    """(Q_BLOCK_SIZE, KV_BLOCK_SIZE) from an int or a pair (block_mask.py:10-14)."""
    if isinstance(BLOCK_SIZE, (int, np.integer)):
        return int(BLOCK_SIZE), int(BLOCK_SIZE)
    return tuple(BLOCK_SIZE)


# ---------------------------------------------------------------------------
# grid helpers (vectorize.py:9-33, 175-253)
# ---------------------------------------------------------------------------


def array_from_coords(shape, fn) -> np.ndarray:
    """result[i, j, ...] = fn(i, j, ...) over ``shape`` (vectorize.py:9-33).

    ``fn`` receives one broadcastable int64 index array per axis."""
    n = len(shape)
    grids = [np.arange(s, dtype=np.int64).reshape((1,) * i + (s,) + (1,) * (n - i - 1))
             for i, s in enumerate(shape)]
    return np.array(np.broadcast_to(np.asarray(fn(*grids)), tuple(shape)))


def nested_fori_loop(lowers, uppers, body_fun, init_val):
    """Nested counted loops (vectorize.py:175-253): level i runs from lowers[i] to
    uppers[i], each an int or a function of the enclosing indices, and
    ``body_fun(i0, i1, ..., val)`` returns the next ``val``."""
    depth = len(lowers)

    def bound(x, idx):
        return int(x(*idx)) if callable(x) else int(x)

    def run(level, idx, val):
        for i in range(bound(lowers[level], idx), bound(uppers[level], idx)):
            if level == depth - 1:
                val = body_fun(*idx, i, val)
            else:
                val = run(level + 1, idx + (i,), val)
        return val

    return run(0, (), init_val)


# ---------------------------------------------------------------------------
# jax indexing semantics for computed indices
# ---------------------------------------------------------------------------


def _read(a: np.ndarray, *idx):
    """a[idx] with jax's gather rule: negative indices count from the end, the
    result is clamped into range."""
    fixed = []
    for ax, i in enumerate(idx):
        n = a.shape[ax]
        i = np.asarray(i, np.int64)
        i = np.where(i < 0, i + n, i)
        fixed.append(np.clip(i, 0, n - 1))
    return a[tuple(fixed)]


def _write_index(i, n):
    """(index, keep) for a write along an axis of length n with jax's scatter
    rule: negative indices count from the end, out-of-range writes are dropped."""
    i = np.asarray(i, np.int64)
    i = np.where(i < 0, i + n, i)
    return np.clip(i, 0, max(n - 1, 0)), (i >= 0) & (i < n)


def _list_entries(B, H, ROWS, num, idx):
    """Every (b, h, row, listed index) of padded per-row lists: row (b, h, i)
    lists idx[b, h, i, j] for j < num[b, h, i] (reads clamped as in jax)."""
    b, h, i = (x.reshape(-1) for x in np.meshgrid(np.arange(B), np.arange(H), np.arange(ROWS),
                                                  indexing="ij"))
    cnt = np.maximum(_read(num, b, h, i).astype(np.int64), 0) if b.size else np.zeros(0, np.int64)
    tot = int(cnt.sum())
    rows = np.repeat(np.arange(b.size), cnt)
    j = np.arange(tot) - np.repeat(np.cumsum(cnt) - cnt, cnt)
    b, h, i = b[rows], h[rows], i[rows]
    return b, h, i, (_read(idx, b, h, i, j).astype(np.int64) if tot else np.zeros(0, np.int64))


def _eval_blocks(mask_mod, b, h, qb, kb, Qb, KVb):
    """mask_mod over the listed tiles: bool [n, Qb, KVb]."""
    out = np.zeros((len(b), Qb, KVb), bool)
    rq = np.arange(Qb, dtype=np.int64)[None, :, None]
    rk = np.arange(KVb, dtype=np.int64)[None, None, :]
    step = max(1, _CHUNK // max(1, Qb * KVb))
    for s in range(0, len(b), step):
        e = slice(s, s + step)
        v = mask_mod(b[e, None, None], h[e, None, None], qb[e, None, None] * Qb + rq,
                     kb[e, None, None] * KVb + rk)
        out[e] = np.broadcast_to(np.asarray(v, bool), out[e].shape)
    return out


# ---------------------------------------------------------------------------
# the descriptor
# ---------------------------------------------------------------------------


@dataclass(frozen=True, eq=False)
class BlockMask:
    """Block-sparse mask (block_mask.py:17-42).  ``kv_num_blocks`` /
    ``kv_indices`` list the PARTIAL tiles of each query-block row, ``full_kv_*``
    the FULL ones; ``q_*`` / ``full_q_*`` are the same per key-block column
    (None when built by ``from_kv_blocks`` without ``generate_q_blocks``)."""

    B: int
    H: int
    Q_LEN: int
    KV_LEN: int
    Q_BLOCK_SIZE: int
    KV_BLOCK_SIZE: int
    kv_num_blocks: np.ndarray                 # int32 [b, h, num_q_blocks]
    kv_indices: np.ndarray                    # int32 [b, h, num_q_blocks, width]
    q_num_blocks: Optional[np.ndarray]        # int32 [b, h, num_kv_blocks]
    q_indices: Optional[np.ndarray]           # int32 [b, h, num_kv_blocks, width]
    full_kv_num_blocks: Optional[np.ndarray]
    full_kv_indices: Optional[np.ndarray]
    full_q_num_blocks: Optional[np.ndarray]
    full_q_indices: Optional[np.ndarray]
    mask_mod: Callable

    # -- element masks -------------------------------------------------------

    def get_mask_for_partial_block(self, b, h, q_block_idx, kv_block_idx) -> np.ndarray:
        """bool [Q_BLOCK_SIZE, KV_BLOCK_SIZE]: mask_mod over one tile (block_mask.py:44-66)."""
        return get_partial_block(self.mask_mod, b, h, q_block_idx, kv_block_idx,
                                 self.Q_BLOCK_SIZE, self.KV_BLOCK_SIZE, self.B, self.H)

    def materialize_mask(self) -> np.ndarray:
        """int32 [B, H, Q_LEN, KV_LEN]: the listed partial tiles filled from
        mask_mod, then the listed full tiles set (block_mask.py:68-129)."""
        Qb, KVb = self.Q_BLOCK_SIZE, self.KV_BLOCK_SIZE
        if self.Q_LEN % Qb or self.KV_LEN % KVb:
            raise ValueError(f"Q_LEN={self.Q_LEN} / KV_LEN={self.KV_LEN} are not multiples of the "
                             f"block sizes ({Qb}, {KVb})")
        NQ, NK = self.Q_LEN // Qb, self.KV_LEN // KVb
        rows = self.kv_num_blocks.shape[-1]
        mask = np.zeros((self.B, self.H, NQ, NK, Qb, KVb), bool)

        b, h, i, kv = _list_entries(self.B, self.H, rows, self.kv_num_blocks, self.kv_indices)
        kv_w, keep = _write_index(kv, NK)
        keep &= i < NQ
        if keep.any():
            b, h, i, kv, kv_w = b[keep], h[keep], i[keep], kv[keep], kv_w[keep]
            mask[b, h, i, kv_w] = _eval_blocks(self.mask_mod, b, h, i, kv, Qb, KVb)

        b, h, i, kv = _list_entries(self.B, self.H, rows, self.full_kv_num_blocks,
                                    self.full_kv_indices)
        kv_w, keep = _write_index(kv, NK)
        keep &= i < NQ
        mask[b[keep], h[keep], i[keep], kv_w[keep]] = True
        return mask.transpose(0, 1, 2, 4, 3, 5).reshape(self.B, self.H, self.Q_LEN,
                                                        self.KV_LEN).astype(np.int32)

    # -- tile-level views ----------------------------------------------------

    def get_full_blocks(self) -> np.ndarray:
        """bool [B, H, rows, cols]: the full tiles (block_mask.py:131-142)."""
        ROWS = self.full_kv_num_blocks.shape[-1]
        COLS = self.full_q_num_blocks.shape[-1]
        return get_dense_from_kv_blocks(self.B, self.H, ROWS, COLS, self.full_kv_num_blocks,
                                        self.full_kv_indices)

    def get_partial_blocks(self) -> np.ndarray:
        """bool [B, H, rows, cols]: the partial tiles (block_mask.py:144-155)."""
        ROWS = self.kv_num_blocks.shape[-1]
        COLS = self.q_num_blocks.shape[-1]
        return get_dense_from_kv_blocks(self.B, self.H, ROWS, COLS, self.kv_num_blocks,
                                        self.kv_indices)

    def to_dense(self) -> np.ndarray:
        """bool [B, H, rows, cols]: tiles that are full or partial (block_mask.py:157-165;
        jax adds boolean arrays as a logical or)."""
        return self.get_full_blocks() | self.get_partial_blocks()

    # -- constructors --------------------------------------------------------

    @classmethod
    def full_mask(cls, B, H, Q_LEN, KV_LEN, BLOCK_SIZE) -> "BlockMask":
        """Every tile full, no q lists (block_mask.py:167-184)."""
        Qb, KVb = extract_block_size(BLOCK_SIZE)
        nk, nq = KV_LEN // KVb, Q_LEN // Qb
        return cls.from_kv_blocks(
            kv_num_blocks=np.zeros((B, H, nq), np.int32),
            kv_indices=np.ones((B, H, nq, 1), np.int32),
            full_kv_num_blocks=np.full((B, H, nq), nk, np.int32),
            full_kv_indices=np.broadcast_to(np.arange(nk, dtype=np.int32), (B, H, nq, nk)),
            BLOCK_SIZE=(Qb, KVb),
            mask_mod=_allow_all,
            seq_lengths=(Q_LEN, KV_LEN),
        )

    @classmethod
    def causal_mask(cls, B, H, Q_LEN, KV_LEN, BLOCK_SIZE) -> "BlockMask":
        """Tiles below the block diagonal full, diagonal tiles partial under
        q >= k (block_mask.py:186-225); classified by block index, as in the
        reference, also when the two block sizes differ."""
        Qb, KVb = extract_block_size(BLOCK_SIZE)
        nk, nq = KV_LEN // KVb, Q_LEN // Qb
        full = np.broadcast_to(np.tri(nq, nk, -1, dtype=bool), (B, H, nq, nk))
        part = np.broadcast_to(np.eye(nq, nk, dtype=bool), (B, H, nq, nk))
        kv_num, kv_idx = get_sparse_kv_data_from_blocks(part)
        q_num, q_idx = get_sparse_q_data_from_blocks(part)
        fkv_num, fkv_idx = get_sparse_kv_data_from_blocks(full)
        fq_num, fq_idx = get_sparse_q_data_from_blocks(full)
        return cls(B, H, Q_LEN, KV_LEN, Qb, KVb, kv_num, kv_idx, q_num, q_idx, fkv_num, fkv_idx,
                   fq_num, fq_idx, _causal)

    @classmethod
    def from_blocks(cls, partial_blocks, full_blocks, BLOCK_SIZE, mask_mod) -> "BlockMask":
        """From dense [b, h, rows, cols] tile classifications; tiles marked in
        both count as full (block_mask.py:227-275)."""
        Qb, KVb = extract_block_size(BLOCK_SIZE)
        partial_blocks = np.asarray(partial_blocks)
        full_blocks = np.asarray(full_blocks)
        B, H = partial_blocks.shape[0], partial_blocks.shape[1]
        partial_blocks = np.where(full_blocks, np.zeros_like(partial_blocks), partial_blocks)
        nq, nk = partial_blocks.shape[2], partial_blocks.shape[3]
        kv_num, kv_idx = get_sparse_kv_data_from_blocks(partial_blocks)
        q_num, q_idx = get_sparse_q_data_from_blocks(partial_blocks)
        fkv_num, fkv_idx = get_sparse_kv_data_from_blocks(full_blocks)
        fq_num, fq_idx = get_sparse_q_data_from_blocks(full_blocks)
        return cls(B, H, nq * Qb, nk * KVb, Qb, KVb, kv_num, kv_idx, q_num, q_idx, fkv_num, fkv_idx,
                   fq_num, fq_idx, mask_mod)

    @classmethod
    def from_kv_blocks(cls, kv_num_blocks, kv_indices, full_kv_num_blocks, full_kv_indices,
                       BLOCK_SIZE, mask_mod, seq_lengths=None,
                       generate_q_blocks=False) -> "BlockMask":
        """From per-row lists (block_mask.py:277-378).  Without ``seq_lengths``,
        Q_LEN = rows x Q_BLOCK_SIZE and KV_LEN = (largest listed key block + 1) x
        KV_BLOCK_SIZE.  ``generate_q_blocks`` rebuilds every list via from_blocks."""
        Qb, KVb = extract_block_size(BLOCK_SIZE)
        kv_num_blocks, kv_indices, full_kv_num_blocks, full_kv_indices = (
            np.asarray(x) for x in (kv_num_blocks, kv_indices, full_kv_num_blocks, full_kv_indices))
        for name, a, nd in (("kv_num_blocks", kv_num_blocks, 3), ("kv_indices", kv_indices, 4),
                            ("full_kv_num_blocks", full_kv_num_blocks, 3),
                            ("full_kv_indices", full_kv_indices, 4)):
            if a.ndim < nd:
                # the reference's "... q -> 1 1 q" rearrange rejects every such input
                raise RuntimeError(f"{name} needs {nd} dimensions [b, h, ...], got shape {a.shape}")
        B, H = kv_num_blocks.shape[0], kv_num_blocks.shape[1]
        if seq_lengths is None:
            Q_LEN = kv_indices.shape[2] * Qb
            top = max(_max_listed(kv_num_blocks, kv_indices, B, H),
                      _max_listed(full_kv_num_blocks, full_kv_indices, B, H))
            KV_LEN = (top + 1) * KVb
        else:
            Q_LEN, KV_LEN = seq_lengths
        if not generate_q_blocks:
            return cls(B, H, Q_LEN, KV_LEN, Qb, KVb, kv_num_blocks, kv_indices, None, None,
                       full_kv_num_blocks, full_kv_indices, None, None, mask_mod)
        nq, nk = Q_LEN // Qb, KV_LEN // KVb
        part = get_dense_from_kv_blocks(B, H, nq, nk, kv_num_blocks, kv_indices)
        full = get_dense_from_kv_blocks(B, H, nq, nk, full_kv_num_blocks, full_kv_indices)
        return cls.from_blocks(part, full, BLOCK_SIZE, mask_mod)

    # -- hand-over to the kernels --------------------------------------------

    def tile_map(self, B: int, Hq: int, Hkv: int, element_head: str = "kv") -> "_bm.TileMap":
        """The kernels' tile map of this mask applied to queries [B, Hq, Q_LEN]
        and keys [B, Hkv, KV_LEN], with the element rule of the reference's
        ``flex_attention`` (attention.py:579-676): the tiles of query head hq
        are the lists of row (b, hq) (of row 0 along an axis the mask has size 1
        on); a full tile allows all its elements, a partial tile those where
        ``mask_mod(b', h', q, k)`` holds, b' / h' being 0 along a broadcast axis
        and h' otherwise the KV head hq // (Hq / Hkv) (attention.py:561-575).
        ``element_head="query"`` evaluates with hq itself instead, which is what
        ``materialize_mask`` and the reference's ``flex_attention_slow`` do
        (attention.py:799-809); the two agree unless Hq > Hkv.

        Raises ValueError where the reference's result is not a mask: a tile
        listed twice in a row (the reference would sum it twice) or a listed
        index outside the key blocks (the reference clamps it)."""
        Qb, KVb = self.Q_BLOCK_SIZE, self.KV_BLOCK_SIZE
        if self.Q_LEN % Qb or self.KV_LEN % KVb:
            raise ValueError("query / key length must be divisible by the block sizes")
        if self.B not in (1, B) or self.H not in (1, Hq):
            raise ValueError(f"block mask is for B={self.B}, H={self.H}; inputs have B={B}, Hq={Hq}")
        NQ, NK = self.Q_LEN // Qb, self.KV_LEN // KVb
        G = Hq // Hkv
        map_b, map_h = self.B, self.H
        # tile classes of the map rows: 0 absent, 1 full, 2 partial
        cls_ = np.zeros((map_b, map_h, NQ, NK), np.int8)
        for kind, num, idx in ((1, self.full_kv_num_blocks, self.full_kv_indices),
                               (2, self.kv_num_blocks, self.kv_indices)):
            b, h, i, kv = _list_entries(map_b, map_h, NQ, num, idx)
            if ((kv < 0) | (kv >= NK)).any():
                raise ValueError(f"block mask lists key block indices outside [0, {NK})")
            if (cls_[b, h, i, kv] != 0).any() or len(np.unique(
                    ((b * map_h + h) * NQ + i) * NK + kv)) != len(kv):
                raise ValueError("block mask lists a tile more than once in a row")
            cls_[b, h, i, kv] = kind
        mask_mod = self.mask_mod
        if element_head not in ("kv", "query"):
            raise ValueError(f"element_head must be 'kv' or 'query', got {element_head!r}")
        if map_h == 1:
            h_elem = np.zeros(1, np.int64)
        else:
            h_elem = np.arange(map_h) // (G if element_head == "kv" else 1)
        nkt = -(-self.KV_LEN // _bm.TILE)

        def strip(q0):
            rows = min(_bm.TILE, self.Q_LEN - q0)
            out = np.zeros((map_b, map_h, _bm.TILE, nkt * _bm.TILE), bool)
            for qb in range(q0 // Qb, -(-(q0 + rows) // Qb)):
                lo, hi = max(q0, qb * Qb), min(q0 + rows, (qb + 1) * Qb)
                c = cls_[:, :, qb]                                        # [map_b, map_h, NK]
                mb, mh, kb = np.nonzero(c)
                for x, y, z in zip(mb, mh, kb):
                    sl = out[x, y, lo - q0:hi - q0, z * KVb:(z + 1) * KVb]
                    if c[x, y, z] == 1:
                        sl[...] = True
                    else:
                        q = np.arange(lo, hi, dtype=np.int64)[:, None]
                        k = np.arange(z * KVb, (z + 1) * KVb, dtype=np.int64)[None, :]
                        sl[...] = np.broadcast_to(np.asarray(
                            mask_mod(np.int64(x), np.int64(h_elem[y]), q, k), bool), sl.shape)
            return out

        return _bm.trace_strips(strip, B, Hq, Hkv, self.Q_LEN, self.KV_LEN, map_b, map_h)


def _allow_all(b, h, q, k):
    return True


def _causal(b, h, q, k):
    return q >= k


def _max_listed(num, idx, B, H):
    """Largest listed index over rows, as the reference computes it
    (block_mask.py:306-332): unlisted columns count as -inf, cast to int32."""
    rows = idx.shape[2]
    col = np.arange(idx.shape[3])
    n = _read(num, *np.meshgrid(np.arange(B), np.arange(H), np.arange(rows), indexing="ij"))
    v = np.where(col < n[..., None], _read(idx, *np.meshgrid(
        np.arange(B), np.arange(H), np.arange(rows), col, indexing="ij")).astype(np.float64), -np.inf)
    m = v.max() if v.size else -np.inf
    return int(m) if np.isfinite(m) else int(np.iinfo(np.int32).min)


# ---------------------------------------------------------------------------
# module functions
# ---------------------------------------------------------------------------


def get_partial_block(mask_mod, b, h, block_q_idx, block_kv_idx, Q_BLOCK_SIZE, KV_BLOCK_SIZE, B,
                      H) -> np.ndarray:
    """bool [Q_BLOCK_SIZE, KV_BLOCK_SIZE]: mask_mod over one tile (block_mask.py:381-408)."""
    q0, k0 = block_q_idx * Q_BLOCK_SIZE, block_kv_idx * KV_BLOCK_SIZE
    return array_from_coords((Q_BLOCK_SIZE, KV_BLOCK_SIZE),
                             lambda q, k: mask_mod(b, h, q0 + q, k0 + k)).astype(bool)


def get_sparse_kv_data_from_blocks(blocks):
    """(num, indices) of a dense [b, h, rows, cols] (or [rows, cols]) tile
    classification: num = count per row (int32), indices = stable argsort of
    -blocks, i.e. the marked columns first, ascending (block_mask.py:411-432)."""
    blocks = np.asarray(blocks).astype(np.int32)
    if blocks.ndim == 2:
        blocks = blocks[None, None]
    num = blocks.sum(axis=-1, dtype=np.int32)
    idx = np.argsort(-blocks, axis=-1, kind="stable").astype(np.int32)
    return num, idx


def get_sparse_q_data_from_blocks(blocks):
    """The per-column lists: get_sparse_kv_data_from_blocks of the transpose
    (block_mask.py:435-451)."""
    blocks = np.asarray(blocks)
    if blocks.ndim != 4:
        raise RuntimeError(f"tile classification needs [b, h, q, kv], got shape {blocks.shape}")
    return get_sparse_kv_data_from_blocks(np.swapaxes(blocks, 2, 3))


def create_block_mask(mask_mod, B, H, Q_LEN, KV_LEN, BLOCK_SIZE) -> BlockMask:
    """Classifies every tile by evaluating ``mask_mod`` on it: all true -> full,
    some true -> partial (block_mask.py:454-498).

    Evaluated once per distinct (b, h): the broadcast shape of ``mask_mod``'s
    result shows which of the two it depends on, as in the kernels' tracer."""
    Qb, KVb = extract_block_size(BLOCK_SIZE)
    nq, nk = Q_LEN // Qb, KV_LEN // KVb
    full = np.zeros((B, H, nq, nk), np.int32)
    part = np.zeros((B, H, nq, nk), np.int32)
    if nq and nk and B and H:
        mb, mh = _bm._probe_dependence(mask_mod, B, H, nq * Qb, nk * KVb)
        b = np.arange(mb, dtype=np.int64)[:, None, None, None]
        h = np.arange(mh, dtype=np.int64)[None, :, None, None]
        k = np.arange(nk * KVb, dtype=np.int64)[None, None, None, :]
        step = max(1, _CHUNK // max(1, mb * mh * Qb * nk * KVb))
        for r0 in range(0, nq, step):
            r1 = min(nq, r0 + step)
            q = np.arange(r0 * Qb, r1 * Qb, dtype=np.int64)[None, None, :, None]
            m = np.broadcast_to(np.asarray(mask_mod(b, h, q, k), bool),
                                (mb, mh, (r1 - r0) * Qb, nk * KVb))
            t = m.reshape(mb, mh, r1 - r0, Qb, nk, KVb)
            a, e = t.all(axis=(3, 5)), t.any(axis=(3, 5))
            full[:, :, r0:r1] = a
            part[:, :, r0:r1] = a ^ e
    return BlockMask.from_blocks(part, full, BLOCK_SIZE, mask_mod)


def get_dense_from_kv_blocks(B, H, NUM_Q_BLOCKS, NUM_KV_BLOCKS, kv_num_blocks,
                             kv_indices) -> np.ndarray:
    """bool [B, H, rows, cols] with the listed tiles set (block_mask.py:501-536)."""
    data = np.zeros((B, H, NUM_Q_BLOCKS, NUM_KV_BLOCKS), bool)
    b, h, i, kv = _list_entries(B, H, NUM_Q_BLOCKS, np.asarray(kv_num_blocks), np.asarray(kv_indices))
    kv_w, keep = _write_index(kv, NUM_KV_BLOCKS)
    data[b[keep], h[keep], i[keep], kv_w[keep]] = True
    return data
