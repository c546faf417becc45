"""Masks in closed form: ``mask_fn(b, h, q, k)`` functions the GPU can classify.

Each constructor returns an ordinary four-argument mask function, valid
anywhere the reference takes ``mask_fn`` (``attention.py:347-357``; it is
called elementwise, with scalars under ``vmap`` there and with broadcast numpy
index arrays here).  The function also carries a :class:`MaskSpec`, and
``masked_attention_via_map`` builds the tile map of such a mask on the GPU
(``mattn_tilemap_classify``, one wave per 128 x 128 tile) instead of
evaluating it element by element on the host -- the host tracer's cost is
B·H·L² evaluations for masks that depend on the batch or head, which is
what ``create_block_mask`` (``block_mask.py:454-498``) pays too.

Families, combined with :func:`intersect`:

* :func:`causal` -- ``q >= k`` (``attention.py:410-415``);
* :func:`window` -- ``q - k <= left`` and ``k - q <= right`` (element level, as
  in the reference tests' sliding-window masks, ``test_mapped_attention.py:1552``);
* :func:`documents` -- ``doc[q] == doc[k]`` for packed sequences, one id array
  for every batch or one per batch;
* :func:`same_residue` -- ``k % period == q % period``, the strided mask of the
  reference's benchmark (``check_attn.py:9-32``, with ``causal``);
* :func:`tile_table` -- a per-128x128-tile table (shared, per head or per batch
  and head): 0 masks the tile, 1 allows every element of it, 2 applies the
  element predicates above (a BlockMask's full and partial tiles,
  ``block_mask.py:17-42``).
"""
from __future__ import annotations

from dataclasses import dataclass, replace
from typing import Optional

import numpy as np

TILE = 128

__all__ = ["MaskSpec", "causal", "window", "documents", "same_residue", "tile_table", "intersect",
           "spec_of"]


@dataclass(frozen=True, eq=False)
class MaskSpec:
    causal: bool = False
    win_left: Optional[int] = None     # q - k <= win_left
    win_right: Optional[int] = None    # k - q <= win_right
    doc_q: Optional[np.ndarray] = None   # int32 [1 or B, Lq]
    doc_k: Optional[np.ndarray] = None   # int32 [1 or B, Lk]
    table: Optional[np.ndarray] = None   # uint8 [1 or B, 1 or H, ceil(Lq/128), ceil(Lk/128)]
    period: Optional[int] = None         # (q - k) % period == 0

    def evaluate(self, b, h, q, k):
        """The mask at broadcast index arrays (or scalars)."""
        b, h, q, k = (np.asarray(x) for x in (b, h, q, k))
        m = np.asarray(True)
        if self.causal:
            m = m & (q >= k)
        if self.win_left is not None:
            m = m & (q - k <= self.win_left)
        if self.win_right is not None:
            m = m & (k - q <= self.win_right)
        if self.doc_q is not None:
            bd = b if self.doc_q.shape[0] > 1 else 0
            m = m & (self.doc_q[bd, q] == self.doc_k[bd, k])
        if self.period is not None:
            m = m & ((q - k) % self.period == 0)
        if self.table is not None:
            tb = b if self.table.shape[0] > 1 else 0
            th = h if self.table.shape[1] > 1 else 0
            tv = self.table[tb, th, q // TILE, k // TILE]
            m = (tv == 1) | ((tv == 2) & m)
        return m

    def map_dims(self, B: int, Hq: int):
        """(map_b, map_h): 1 where the mask is the same for every batch / head."""
        nb = max(self.doc_q.shape[0] if self.doc_q is not None else 1,
                 self.table.shape[0] if self.table is not None else 1)
        nh = self.table.shape[1] if self.table is not None else 1
        return (B if nb > 1 else 1), (Hq if nh > 1 else 1)

    def check(self, B: int, Hq: int, Lq: int, Lk: int):
        """ValueError unless the spec's arrays fit a (B, Hq, Lq, Lk) problem."""
        if self.doc_q is not None:
            if self.doc_q.shape[1] != Lq or self.doc_k.shape[1] != Lk:
                raise ValueError(f"document ids of lengths {self.doc_q.shape[1]}/{self.doc_k.shape[1]} "
                                 f"for query/key lengths {Lq}/{Lk}")
            if self.doc_q.shape[0] not in (1, B):
                raise ValueError(f"document ids for {self.doc_q.shape[0]} batches, B = {B}")
        if self.table is not None:
            nb, nh, nq, nk = self.table.shape
            want = (-(-Lq // TILE), -(-Lk // TILE))
            if (nq, nk) != want:
                raise ValueError(f"tile table of {nq}x{nk} tiles, the problem has {want[0]}x{want[1]}")
            if nb not in (1, B) or nh not in (1, Hq):
                raise ValueError(f"tile table for {nb} batches x {nh} heads, problem has {B} x {Hq}")


def _fn(spec: MaskSpec):
    def mask_fn(b, h, q, k):
        return spec.evaluate(b, h, q, k)

    mask_fn._mattn_spec = spec
    return mask_fn


def spec_of(mask_fn) -> Optional[MaskSpec]:
    """The closed form a mask function carries, or None (an arbitrary callable)."""
    return getattr(mask_fn, "_mattn_spec", None)


def _frozen(a, dtype):
    a = np.array(a, dtype=dtype, copy=True)
    a.setflags(write=False)
    return a


def causal():
    """q >= k."""
    return _fn(MaskSpec(causal=True))


def window(left: Optional[int] = None, right: Optional[int] = 0):
    """q - k <= left and k - q <= right (None: unbounded on that side)."""
    for v in (left, right):
        if v is not None and (int(v) != v or v < 0):
            raise ValueError(f"window bounds must be non-negative integers or None, got {v}")
    return _fn(MaskSpec(win_left=None if left is None else int(left),
                        win_right=None if right is None else int(right)))


def documents(doc_ids, doc_ids_k=None):
    """doc_ids[b, q] == doc_ids_k[b, k]; ids of shape [L] (every batch) or [B, L].
    ``doc_ids_k`` defaults to ``doc_ids`` (self-attention over packed documents)."""
    dq = np.asarray(doc_ids)
    dk = dq if doc_ids_k is None else np.asarray(doc_ids_k)
    if dq.ndim == 1:
        dq = dq[None]
    if dk.ndim == 1:
        dk = dk[None]
    if dq.ndim != 2 or dk.ndim != 2 or dq.shape[0] != dk.shape[0]:
        raise ValueError("document ids must be [L] or [B, L], the same batch count for q and k")
    if not (np.issubdtype(dq.dtype, np.integer) and np.issubdtype(dk.dtype, np.integer)):
        raise ValueError("document ids must be integers")
    for a in (dq, dk):
        if a.size and (a.min() < np.iinfo(np.int32).min or a.max() > np.iinfo(np.int32).max):
            raise ValueError("document ids must fit in int32")
    return _fn(MaskSpec(doc_q=_frozen(dq, np.int32), doc_k=_frozen(dk, np.int32)))


def same_residue(period: int):
    """k % period == q % period, i.e. (q - k) % period == 0: every period-th
    key (with :func:`causal`, the mask of ``check_attn.py:9-32``)."""
    if int(period) != period or period < 1 or period > 2**31 - 1:
        raise ValueError(f"period must be a positive int32, got {period}")
    return _fn(MaskSpec(period=int(period)))


def tile_table(table):
    """Per-128x128-tile table of shape [nqt, nkt], [H, nqt, nkt] or [B, H, nqt, nkt]:
    0 = no element, 1 = every element, 2 = the other predicates of the mask
    (booleans: True = 2)."""
    t = np.asarray(table)
    if t.dtype == bool:
        t = t.astype(np.uint8) * 2
    if t.ndim not in (2, 3, 4):
        raise ValueError("tile table must have 2, 3 or 4 dimensions")
    t = t.reshape((1,) * (4 - t.ndim) + t.shape)
    if t.size and (t.min() < 0 or t.max() > 2):
        raise ValueError("tile table entries must be 0, 1 or 2")
    return _fn(MaskSpec(table=_frozen(t, np.uint8)))


def intersect(*mask_fns):
    """The AND of closed-form masks."""
    specs = [spec_of(m) for m in mask_fns]
    if not specs or any(s is None for s in specs):
        raise ValueError("intersect takes masks made by jaxmodules_amd.masks")
    out = MaskSpec()
    for s in specs:
        kw = {}
        if s.causal:
            kw["causal"] = True
        for side in ("win_left", "win_right"):
            v = getattr(s, side)
            if v is not None:
                cur = getattr(out, side)
                kw[side] = v if cur is None else min(cur, v)
        if s.period is not None:
            # both residue classes: modulo the least common multiple
            p = s.period if out.period is None else int(np.lcm(out.period, s.period))
            if p > 2**31 - 1:
                raise ValueError("the combined period exceeds int32")
            kw["period"] = p
        for name in ("doc_q", "table"):
            if getattr(s, name) is not None:
                if getattr(out, name) is not None:
                    raise ValueError(f"at most one {'document' if name == 'doc_q' else 'tile table'} "
                                     "mask per intersection")
                kw[name] = getattr(s, name)
                if name == "doc_q":
                    kw["doc_k"] = s.doc_k
        out = replace(out, **kw)
    return _fn(out)
