"""Host-side tracer: turns the reference's ``mask_fn`` into the kernels' tile map.

The reference evaluates ``mask_fn(b, h, q, k)`` element by element inside every
(query block, key block) step and multiplies the scores by it, visiting every
key block (``/root/reference/jaxmodules/attention.py:52-105,133-177``).  Its
``block_mask.py`` classifies tiles as empty / full / partial
(``create_block_mask``, block_mask.py:454-498), but only ``flex_attention``
consumes that.  Here the two are joined: the effective mask of a call --
``mask_fn`` AND the window's visited key blocks (attention.py:161-167,199-204)
AND the unpadded range (attention.py:426-437) -- is traced once on the host
into 128 x 128 tiles:

* empty tiles are dropped (the kernels never visit them);
* full tiles are listed with mask id -1 (no per-element work);
* partial tiles carry packed element bitmasks, de-duplicated by content
  (all diagonal tiles of a causal mask share one mask).

``mask_fn`` is called with numpy index arrays that broadcast against each
other (b: [B,1,1,1], h: [1,H,1,1], q: [1,1,Q,1], k: [1,1,1,K]); the reference
calls it with scalars under nested ``vmap`` (vectorize.py:407-527), so any
elementwise function of the indices works in both.  The shape of the result
shows whether the mask depends on b and h; a mask that does not is traced once
and broadcast (``map_b == 1`` / ``map_h == 1``), like the B/H arguments of the
reference's ``create_block_mask``.
"""
from __future__ import annotations

import ctypes
import os
from dataclasses import dataclass, field
from typing import Callable, Optional, Tuple

import numpy as np

from .masks import MaskSpec, spec_of

TILE = 128
NUM_XCD = 8  # MI355X: 8 accelerator complex dies, workgroups dispatched round-robin


# ---------------------------------------------------------------------------
# call canonicalisation (attention.py:385-437 and :195-217)
# ---------------------------------------------------------------------------


@dataclass
class Plan:
    B: int
    N: int               # query length
    L: int               # key length
    Hq: int
    Hkv: int
    d: int
    bs: int              # the reference's block size (query and key blocks)
    Npad: int            # padded lengths the reference works on
    Lpad: int
    mask4: Callable      # canonical 4-argument mask (b, h, q, k)
    window: Optional[Tuple[int, int]]  # (left blocks, right blocks) or None
    squeeze_batch: bool  # inputs were 3-D


def canonical_mask(is_causal: bool, mask_fn):
    """attention.py:404-419: 3-argument masks ignore b; causal is q >= k."""
    if mask_fn is not None and mask_fn.__code__.co_argcount == 3:
        three = mask_fn
        mask_fn = lambda b, h, q, k: three(h, q, k)  # noqa: E731
    if is_causal and mask_fn is not None:
        raise ValueError("cannot specify both 'is_causal' and 'mask_fn'!")
    if is_causal:
        mask_fn = _causal
    if mask_fn is None:
        mask_fn = _everything
    return mask_fn


def _causal(b, h, q, k):
    return q >= k


def _everything(b, h, q, k):
    return True


_causal._mattn_spec = MaskSpec(causal=True)
_everything._mattn_spec = MaskSpec()


def make_plan(q_shape, k_shape, v_shape, *, is_causal=False, mask_fn=None, block_size=None,
              window_size=None) -> Plan:
    """Validation and set-up with the reference's exception types.

    attention.py:385-391 (ndim -> ValueError), :394-399 (3-D inputs gain a batch
    dim), :404-419 (mask), :421-437 (padding to a block multiple: Q by
    bs - N % bs and K/V by bs - L % bs, a whole extra block when L % bs == 0),
    :195-217 (block size, window blocks, shape asserts -> AssertionError).
    """
    for name, s in (("K", k_shape), ("Q", q_shape), ("V", v_shape)):
        if len(s) not in (3, 4):
            raise ValueError(f"{name} must have 3 or 4 dimensions")
    assert len(k_shape) == len(q_shape) and len(v_shape) == len(q_shape), \
        "Q, K, and V must have the same number of dimensions"
    squeeze = len(q_shape) == 3
    if squeeze:
        q_shape, k_shape, v_shape = (1, *q_shape), (1, *k_shape), (1, *v_shape)
    mask4 = canonical_mask(is_causal, mask_fn)
    assert k_shape[0] == q_shape[0] == v_shape[0], "Q, K, and V must have the same batch dimension"
    B, N, Hq, dq = q_shape
    _, L, Hk, d = k_shape
    _, Lv, Hv, dv = v_shape
    Npad, Lpad = N, L
    if block_size is not None and N % block_size != 0:
        Npad = N + block_size - N % block_size
        Lpad = L + block_size - L % block_size
    bs = Npad if block_size is None else block_size
    assert d == dq and Lv == L and dv == d, \
        f"shape mismatch in K {tuple(k_shape)}, Q {tuple(q_shape)} and V {tuple(v_shape)}"
    assert Hq % Hk == 0, "Hq must be divisible by Hk"
    assert Hv == Hk, "Hv must be equal to Hk"
    if Lpad % bs != 0:
        # the reference's rearrange of K into blocks of the query block size fails here
        raise RuntimeError(f"key length {Lpad} is not a multiple of the block size {bs}")
    window = None
    if window_size is not None:
        left, right = window_size
        lwb = (left + bs - 1) // bs
        rwb = 1 + (right + bs - 1) // bs
        if lwb + rwb > Lpad // bs:
            # lax.dynamic_slice_in_dim rejects a slice longer than the operand
            raise TypeError(f"window of {lwb + rwb} key blocks exceeds the {Lpad // bs} blocks present")
        window = (lwb, rwb)
    return Plan(B, N, L, Hq, Hk, d, bs, Npad, Lpad, mask4, window, squeeze)


def window_key_range(plan: Plan, q: np.ndarray):
    """[lo, hi) key range each query's block scans (attention.py:160-167).

    The scan covers ``lwb + rwb`` key blocks starting at max(0, i - lwb), and
    ``dynamic_slice_in_dim`` clamps that start into [0, nk - size]."""
    lwb, rwb = plan.window
    nk = plan.Lpad // plan.bs
    i = q // plan.bs
    start = np.minimum(np.maximum(0, i - lwb), nk - (lwb + rwb))
    return start * plan.bs, (start + lwb + rwb) * plan.bs


# ---------------------------------------------------------------------------
# tile map
# ---------------------------------------------------------------------------


@dataclass
class TileMap:
    B: int
    Hq: int
    Hkv: int
    Lq: int
    Lk: int
    map_b: int
    map_h: int
    nqt: int
    nkt: int
    row_ptr: np.ndarray     # int32 [map_b*map_h*nqt + 1]
    row_ent: np.ndarray     # int32 [nnz, 2] (key tile, mask id)
    col_ptr: np.ndarray     # int32 [map_b*map_h*nkt + 1]
    col_ent: np.ndarray     # int32 [nnz, 2] (query tile, mask id)
    col_row: np.ndarray     # int32 [nnz]: index in row_ent of each col_ent entry (same tile)
    kv_desc: np.ndarray     # int32 [len(kv_order), 8]: per dK/dV launch slot (_kv_desc)
    row_bits: np.ndarray    # uint64 [n_masks, 2, 128]: [m, w, q] bit j = key 64w + j allowed
    col_bits: np.ndarray    # uint64 [n_masks, 2, 128]: [m, w, k] bit j = query 64w + j allowed
    q_order: np.ndarray     # int32 launch order of (b, h, query tile) items
    kv_order: np.ndarray    # int32 launch order of (b, kv head, key tile) items
    pairs: int              # allowed (b, h, q, k) positions over all B x Hq
    n_full: int = 0         # present tiles of each kind, over the (broadcast) map
    n_partial: int = 0
    trace_seconds: float = 0.0
    device: dict = field(default_factory=dict, repr=False)

    @property
    def nnz(self) -> int:
        return int(self.row_ent.shape[0])

    @property
    def n_masks(self) -> int:
        return int(self.row_bits.shape[0])

    def states(self) -> np.ndarray:
        """int8 [map_b, map_h, nqt, nkt]: 0 skipped, 1 full, 2 partial."""
        st = np.zeros((self.map_b * self.map_h * self.nqt, self.nkt), np.int8)
        rows = np.repeat(np.arange(self.map_b * self.map_h * self.nqt), np.diff(self.row_ptr))
        st[rows, self.row_ent[:, 0]] = np.where(self.row_ent[:, 1] < 0, 1, 2)
        return st.reshape(self.map_b, self.map_h, self.nqt, self.nkt)

    def dense(self) -> np.ndarray:
        """The traced mask as bool [map_b, map_h, Lq, Lk] (for checking)."""
        out = np.zeros((self.map_b * self.map_h * self.nqt, TILE, self.nkt * TILE), bool)
        rows = np.repeat(np.arange(self.map_b * self.map_h * self.nqt), np.diff(self.row_ptr))
        for r, (kt, mid) in zip(rows, self.row_ent):
            if mid < 0:
                out[r, :, kt * TILE:(kt + 1) * TILE] = True
            else:
                bits = unpack_tile(self.row_bits[mid])
                out[r, :, kt * TILE:(kt + 1) * TILE] = bits
        out = out.reshape(self.map_b, self.map_h, self.nqt * TILE, self.nkt * TILE)
        return out[:, :, :self.Lq, :self.Lk]


def unpack_tile(words: np.ndarray) -> np.ndarray:
    """bool [128, 128] of one tile mask stored as uint64 [2, 128] ([half][row])."""
    w = np.ascontiguousarray(np.asarray(words, np.uint64).T)          # [row, half]
    return np.unpackbits(w.view(np.uint8).reshape(TILE, 16), axis=1, bitorder="little").astype(bool)


def _probe_dependence(mask4, B, Hq, N, L):
    """Which of (b, h) the mask's value can depend on, read off the broadcast
    shape of one small evaluation."""
    b = np.arange(B, dtype=np.int64)[:, None, None, None]
    h = np.arange(Hq, dtype=np.int64)[None, :, None, None]
    q = np.arange(min(N, 4), dtype=np.int64)[None, None, :, None]
    k = np.arange(min(L, 4), dtype=np.int64)[None, None, None, :]
    shape = np.shape(np.asarray(mask4(b, h, q, k)))
    shape = (1,) * (4 - len(shape)) + tuple(shape)
    return (B if shape[0] != 1 else 1), (Hq if shape[1] != 1 else 1)


def _strip_mask(plan: Plan, map_b, map_h, q0, nkt):
    """Effective mask of query rows [q0, q0+128): bool [map_b, map_h, 128, nkt*128]."""
    rows = min(TILE, plan.N - q0)
    b = np.arange(map_b, dtype=np.int64)[:, None, None, None]
    h = np.arange(map_h, dtype=np.int64)[None, :, None, None]
    q = np.arange(q0, q0 + rows, dtype=np.int64)[None, None, :, None]
    k = np.arange(plan.L, dtype=np.int64)[None, None, None, :]
    m = np.broadcast_to(np.asarray(plan.mask4(b, h, q, k), dtype=bool), (map_b, map_h, rows, plan.L))
    if plan.window is not None:
        lo, hi = window_key_range(plan, q[0, 0, :, 0])
        kk = k[0, 0]
        m = m & ((kk >= lo[:, None]) & (kk < hi[:, None]))[None, None]
    out = np.zeros((map_b, map_h, TILE, nkt * TILE), bool)
    out[:, :, :rows, :plan.L] = m
    return out


# Groups an XCD works on at once.  With all of an XCD's groups interleaved
# (cfg2: 16 heads, 32 MB of K/V against a 4 MB L2) every kernel re-fetched
# more; blocks of 4 measured fastest on cfg2 (forward -5%, dK/dV -6%, dQ -1.5%
# against interleaving all 16; blocks of 1, 2, 3, 6 and 8 in between), and
# shapes with at most 4 groups per XCD (the target shape, cfg3-5) are unchanged.
# On the target shape (4 groups per XCD) blocks of 1 and 2 measured slower:
# step -3.1% and -0.6%, dQ +15% and +6%.
HEADS_AT_ONCE = 4


def _lpt_xcd_order(weights: np.ndarray, groups: np.ndarray) -> np.ndarray:
    """Launch order of work items: items of one group (a (b, head) pair) are
    kept on one XCD (workgroup i runs on XCD i % 8, so a group's K/V stay in
    that die's L2).  An XCD takes its groups HEADS_AT_ONCE at a time -- group g
    is the (g // 8)-th of its XCD, in block (g // 8) // HEADS_AT_ONCE -- and
    inside a block the heaviest items go first (longest processing time
    first).  With fewer groups than XCDs (a single head, say), each group is
    split round-robin over NUM_XCD // groups XCDs instead, so that every die
    has work.  Idle slots are -1."""
    groups = np.asarray(groups)
    ngroups = int(groups.max()) + 1 if groups.size else 0
    if 0 < ngroups < NUM_XCD:
        spread = NUM_XCD // ngroups
        by_group = np.argsort(groups, kind="stable")
        first = np.searchsorted(groups[by_group], np.arange(ngroups))
        rank = np.empty(groups.size, np.int64)
        rank[by_group] = np.arange(groups.size) - first[groups[by_group]]   # index within the group
        groups = groups * spread + rank % spread
    bins = [[] for _ in range(NUM_XCD)]
    block = (groups // NUM_XCD) // HEADS_AT_ONCE
    order = np.lexsort((np.arange(len(weights)), -np.asarray(weights), block))  # block, heavy first, stable
    for it in order:
        bins[int(groups[it]) % NUM_XCD].append(int(it))
    width = max(len(b) for b in bins)
    out = np.full((width, NUM_XCD), -1, np.int32)
    for x, b in enumerate(bins):
        out[:len(b), x] = b
    return out.reshape(-1)


def trace(plan: Plan) -> TileMap:
    """Traces the effective mask of ``plan`` into a TileMap."""
    map_b, map_h = _probe_dependence(plan.mask4, plan.B, plan.Hq, plan.N, plan.L)
    nkt = -(-plan.L // TILE)
    return trace_strips(lambda q0: _strip_mask(plan, map_b, map_h, q0, nkt), plan.B, plan.Hq,
                        plan.Hkv, plan.N, plan.L, map_b, map_h)


def _classify_strip(strip, qt, map_b, map_h, nkt):
    """One query strip's present tiles: (pairs, map row / batch / head indices,
    key tiles, full flags, packed row and column bits of the partial tiles)."""
    m = strip(qt * TILE)
    assert m.shape == (map_b, map_h, TILE, nkt * TILE), m.shape
    pairs = int(np.count_nonzero(m))
    t = m.reshape(map_b, map_h, TILE, nkt, TILE)
    anyb = t.any(axis=(2, 4))
    allb = t.all(axis=(2, 4))
    mb, mh, kt = np.nonzero(anyb)
    full = allb[mb, mh, kt]
    part = np.nonzero(~full)[0]
    rb = cb = None
    if len(part):
        tiles = t[mb[part], mh[part], :, kt[part], :]          # [P, 128 q, 128 k]
        rb = np.ascontiguousarray(np.packbits(tiles, axis=2, bitorder="little")).view(np.uint64)
        cb = np.ascontiguousarray(np.packbits(tiles.transpose(0, 2, 1), axis=2,
                                              bitorder="little")).view(np.uint64)
        # [P, 128 rows, 2 words] -> [P, 2 words, 128 rows]: a wave's 32 rows of one
        # 64-wide half are then one contiguous 256-byte block
        rb = np.ascontiguousarray(rb.transpose(0, 2, 1))
        cb = np.ascontiguousarray(cb.transpose(0, 2, 1))
    return pairs, mb, mh, kt, full, part, rb, cb


# host threads for trace_strips (numpy releases the GIL in the array work)
TRACE_THREADS = max(1, min(16, os.cpu_count() or 1))


def trace_strips(strip, B, Hq, Hkv, N, L, map_b, map_h) -> TileMap:
    """TileMap of the mask whose query rows [q0, q0+128) ``strip(q0)`` returns as
    bool [map_b, map_h, 128, nkt*128] (False beyond N and L); map_b / map_h are
    1 where the mask is the same for every batch / head.  The strips are
    classified on TRACE_THREADS threads and merged in strip order, so the map
    (mask numbering included) does not depend on the thread count."""
    import time
    from concurrent.futures import ThreadPoolExecutor

    t0 = time.perf_counter()
    nqt, nkt = -(-N // TILE), -(-L // TILE)

    masks: dict = {}
    row_bits, col_bits = [], []
    ent_row, ent_kt, ent_mid = [], [], []   # map row index, key tile, mask id
    pairs_map = 0
    n_full = n_partial = 0
    work = lambda qt: _classify_strip(strip, qt, map_b, map_h, nkt)
    threads = min(TRACE_THREADS, nqt)
    if threads > 1:
        ex = ThreadPoolExecutor(threads)
        results = ex.map(work, range(nqt))
    else:
        ex, results = None, map(work, range(nqt))
    try:
        for qt, (pairs, mb, mh, kt, full, part, rb, cb) in enumerate(results):
            pairs_map += pairs
            if len(kt) == 0:
                continue
            mids = np.full(len(kt), -1, np.int64)
            for i, p in enumerate(part):
                key = rb[i].tobytes()
                mid = masks.get(key)
                if mid is None:
                    mid = len(row_bits)
                    masks[key] = mid
                    row_bits.append(rb[i])
                    col_bits.append(cb[i])
                mids[p] = mid
            n_full += int(full.sum())
            n_partial += int((~full).sum())
            ent_row.append((mb * map_h + mh) * nqt + qt)
            ent_kt.append(kt)
            ent_mid.append(mids)
    finally:
        if ex is not None:
            ex.shutdown()

    if ent_row:
        r = np.concatenate(ent_row)
        kt = np.concatenate(ent_kt)
        mid = np.concatenate(ent_mid)
    else:
        r = kt = mid = np.zeros(0, np.int64)
    rb = np.stack(row_bits) if row_bits else np.zeros((0, 2, TILE), np.uint64)
    cb = np.stack(col_bits) if col_bits else np.zeros((0, 2, TILE), np.uint64)
    return _assemble(B, Hq, Hkv, N, L, map_b, map_h, r, kt, mid, rb, cb, pairs_map, n_full,
                     n_partial, t0)


def _assemble(B, Hq, Hkv, N, L, map_b, map_h, r, kt, mid, rb, cb, pairs_map, n_full, n_partial,
              t0) -> TileMap:
    """TileMap from its present tiles: map row r = (mb * map_h + mh) * nqt + qt,
    key tile kt and mask id (-1 full) of each, and the distinct masks' bits."""
    import time

    nqt, nkt = -(-N // TILE), -(-L // TILE)
    nmap = map_b * map_h
    o = np.lexsort((kt, r))                 # rows ascending, key tiles ascending
    r, kt, mid = r[o], kt[o], mid[o]
    row_ptr = np.zeros(nmap * nqt + 1, np.int64)
    np.cumsum(np.bincount(r, minlength=nmap * nqt), out=row_ptr[1:])
    row_ent = np.stack([kt, mid], axis=1).astype(np.int32).reshape(-1, 2)

    mapi, qt_of = r // nqt, r % nqt
    c = mapi * nkt + kt
    oc = np.lexsort((qt_of, c))             # columns ascending, query tiles ascending
    col_ptr = np.zeros(nmap * nkt + 1, np.int64)
    np.cumsum(np.bincount(c, minlength=nmap * nkt), out=col_ptr[1:])
    col_ent = np.stack([qt_of[oc], mid[oc]], axis=1).astype(np.int32).reshape(-1, 2)
    col_row = oc.astype(np.int32)           # the row-ordered index of each column entry

    # launch order (weights = present tiles per work item, +1 for the epilogue)
    row_cnt = np.diff(row_ptr).reshape(map_b, map_h, nqt)
    col_cnt = np.diff(col_ptr).reshape(map_b, map_h, nkt)
    bi = np.arange(B) % map_b
    hi = np.arange(Hq) % map_h
    qw = row_cnt[bi][:, hi].reshape(B * Hq * nqt) + 1                  # item (b*Hq + h)*nqt + qt
    G = Hq // Hkv
    # The query heads of one GQA group read the same K/V: their items share an
    # XCD (group (b*Hq + h) // G = b*Hkv + h // G), so each K/V tile is fetched
    # into one L2 -- unless there are fewer such groups than XCDs, when the
    # per-head groups spread the work over more dies.
    qgroups = np.repeat(np.arange(B * Hq) // (G if B * Hkv >= NUM_XCD else 1), nqt)
    cc = col_cnt[bi][:, hi]                                            # [B, Hq, nkt]
    kvw = cc.reshape(B, Hkv, G, nkt).sum(axis=2).reshape(B * Hkv * nkt) + 1
    kvgroups = np.repeat(np.arange(B * Hkv), nkt)
    q_order = _lpt_xcd_order(qw, qgroups)
    kv_order = _lpt_xcd_order(kvw, kvgroups)
    kv_desc = _kv_desc(kv_order, col_ptr, col_ent, col_row, B, Hq, Hkv, nkt, map_b, map_h)

    pairs = pairs_map * (B // map_b) * (Hq // map_h)
    return TileMap(B, Hq, Hkv, N, L, map_b, map_h, nqt, nkt,
                   row_ptr.astype(np.int32), row_ent, col_ptr.astype(np.int32), col_ent, col_row, kv_desc,
                   np.ascontiguousarray(rb), np.ascontiguousarray(cb), q_order, kv_order, pairs,
                   n_full=n_full, n_partial=n_partial, trace_seconds=time.perf_counter() - t0)


def _kv_desc(kv_order, col_ptr, col_ent, col_row, B, Hq, Hkv, nkt, map_b, map_h) -> np.ndarray:
    """Per dK/dV launch slot, what the kernel's first loads need, in one row:
    (item, first query head g of the GQA group with entries in the column,
    that head's first column entry e and its end, sub-blocks of the whole
    column (2 per entry over the group's heads), and entry e's query tile, mask
    id and row-entry index); (-1, 0, ...) for idle slots and zeros after the
    item for an empty column."""
    G = Hq // Hkv
    it = np.asarray(kv_order, np.int64)
    valid = it >= 0
    i = np.where(valid, it, 0)
    kt, bhk = i % nkt, i // nkt
    hk, b = bhk % Hkv, bhk // Hkv
    cp = np.asarray(col_ptr, np.int64)
    mcs = np.stack([((b % map_b) * map_h + (hk * G + g) % map_h) * nkt + kt for g in range(G)], axis=1)
    cnt = cp[mcs + 1] - cp[mcs]                                   # [slots, G]
    tot = 2 * cnt.sum(axis=1)
    lg0 = np.argmax(cnt > 0, axis=1)                              # 0 when the column is empty
    mc0 = mcs[np.arange(len(it)), lg0]
    e0, lend0 = cp[mc0], cp[mc0 + 1]
    has = valid & (tot > 0)
    ent = np.asarray(col_ent, np.int64).reshape(-1, 2)
    crow = np.asarray(col_row, np.int64)
    ec = np.where(has, e0, 0)
    qt0 = np.where(has, ent[ec, 0] if len(ent) else 0, 0)
    m0 = np.where(has, ent[ec, 1] if len(ent) else 0, 0)
    r0 = np.where(has, crow[ec] if len(crow) else 0, 0)
    d = np.stack([np.where(valid, it, -1), lg0, e0, lend0, tot, qt0, m0, r0], axis=1)
    d[~has, 1:] = 0
    return np.ascontiguousarray(d.astype(np.int32))


def device_trace(plan: Plan, device) -> TileMap:
    """The TileMap of ``trace(plan)``, built on the GPU for a mask in closed form
    (``plan.mask4`` made by ``jaxmodules_amd.masks``, or causal / no mask).

    ``mattn_tilemap_classify`` evaluates every tile on the device (one wave per
    tile) and returns per tile its state, allowed-element count and a 128-bit
    hash of a partial tile's bits.  The host numbers the distinct partial
    masks in the order the host tracer meets them (query tile, map row, key
    tile) -- de-duplicated by hash -- and assembles the lists with the same code
    as ``trace``; ``mattn_tilemap_bits`` then writes the distinct masks and
    checks every partial tile against the mask its hash picked (a collision
    raises).  The result equals ``trace(plan)`` array for array."""
    import time

    import torch

    from . import _lib

    spec = spec_of(plan.mask4)
    if spec is None:
        raise ValueError("device_trace needs a mask made by jaxmodules_amd.masks (or causal / None)")
    t0 = time.perf_counter()
    B, Hq, N, L = plan.B, plan.Hq, plan.N, plan.L
    spec.check(B, Hq, N, L)
    map_b, map_h = spec.map_dims(B, Hq)
    nqt, nkt = -(-N // TILE), -(-L // TILE)
    nmap = map_b * map_h
    lib = _lib.load()
    dev = torch.device(device)
    keep = []

    def up(a):
        t = torch.from_numpy(np.array(a, copy=True, order="C")).to(dev)
        keep.append(t)
        return t.data_ptr()

    ms = _lib.MattnMaskspec(causal=int(spec.causal),
                            win_left=-1 if spec.win_left is None else min(spec.win_left, 2**31 - 2),
                            win_right=-1 if spec.win_right is None else min(spec.win_right, 2**31 - 2))
    if spec.doc_q is not None:
        ms.doc_b = spec.doc_q.shape[0] if map_b > 1 else 1
        ms.doc_q = up(spec.doc_q[:ms.doc_b])
        ms.doc_k = up(spec.doc_k[:ms.doc_b])
    if spec.table is not None:
        ms.tab_b, ms.tab_h = spec.table.shape[0], spec.table.shape[1]
        ms.tiles = up(spec.table)
    if plan.window is not None:
        ms.blk_size, ms.blk_left, ms.blk_right = plan.bs, plan.window[0], plan.window[1]
        ms.blk_nk = plan.Lpad // plan.bs
    if spec.period is not None and spec.period > 1:
        ms.res_period = spec.period
    nt = nmap * nqt * nkt
    state = torch.empty(nt, dtype=torch.int8, device=dev)
    count = torch.empty(nt, dtype=torch.int32, device=dev)
    hsh = torch.empty(2 * nt, dtype=torch.int64, device=dev)
    stream = torch.cuda.current_stream(dev).cuda_stream
    args = (ctypes.byref(ms), N, L, map_b, map_h)
    _lib.check(lib.mattn_tilemap_classify(*args, state.data_ptr(), count.data_ptr(), hsh.data_ptr(),
                                          stream), "mattn_tilemap_classify")
    st = state.cpu().numpy().reshape(nmap, nqt, nkt)
    cnt = count.cpu().numpy()
    hv = hsh.cpu().numpy().view(np.uint64).reshape(nmap, nqt, nkt, 2)

    # partial tiles in the host tracer's order of discovery: query tile, map row, key tile
    qp, mp, kp = np.nonzero(st.transpose(1, 0, 2) == 2)
    tidx = (mp * nqt + qp) * nkt + kp
    if len(tidx):
        h = np.ascontiguousarray(hv[mp, qp, kp]).view(np.dtype((np.void, 16))).reshape(-1)
        _, first, inv = np.unique(h, return_index=True, return_inverse=True)
        rank = np.empty(len(first), np.int64)
        rank[np.argsort(first)] = np.arange(len(first))
        pmid = rank[inv.reshape(-1)]
        n_masks = len(first)
        reps = np.stack([tidx[np.sort(first)], np.arange(n_masks)], axis=1).astype(np.int32)
        allp = np.stack([tidx, pmid], axis=1).astype(np.int32)
        rbits = torch.empty(n_masks * 2 * TILE, dtype=torch.int64, device=dev)
        cbits = torch.empty_like(rbits)
        bad = torch.zeros(1, dtype=torch.int32, device=dev)
        for lst, write in ((reps, 1), (allp, 0)):
            _lib.check(lib.mattn_tilemap_bits(*args, up(lst.reshape(-1)), len(lst), n_masks, write,
                                              rbits.data_ptr(), cbits.data_ptr(), bad.data_ptr(),
                                              stream), "mattn_tilemap_bits")
        if int(bad.item()) != 0:
            raise RuntimeError("tile-map hash collision: two different partial tiles hashed alike")
        rb = rbits.cpu().numpy().view(np.uint64).reshape(n_masks, 2, TILE)
        cb = cbits.cpu().numpy().view(np.uint64).reshape(n_masks, 2, TILE)
    else:
        pmid = np.zeros(0, np.int64)
        rb = cb = np.zeros((0, 2, TILE), np.uint64)

    # present tiles: map row, key tile, mask id
    mm, qq, kk = np.nonzero(st)
    mid = np.full(len(mm), -1, np.int64)
    flat = (mm * nqt + qq) * nkt + kk
    if len(tidx):
        pos = np.searchsorted(flat, tidx)      # flat is ascending; every partial tile is in it
        mid[pos] = pmid
    r = mm * nqt + qq
    n_partial = len(tidx)
    n_full = len(mm) - n_partial
    pairs_map = int(cnt.astype(np.int64).sum())
    return _assemble(B, Hq, plan.Hkv, N, L, map_b, map_h, r.astype(np.int64), kk.astype(np.int64),
                     mid, np.ascontiguousarray(rb), np.ascontiguousarray(cb), pairs_map, n_full,
                     n_partial, t0)


def flops(tm: TileMap, d: int):
    """Algorithmic FLOPs counted on unmasked pairs: fwd 4*d*pairs, bwd 10*d*pairs."""
    return 4 * d * tm.pairs, 10 * d * tm.pairs
