"""The stored-dS backward (MATTN_BWD_DS, GPU): the dK/dV kernel leaves dS of
every present tile in the workspace and the dQ kernel computes dQ = dS K from
it instead of recomputing S and dP.

* The stored blocks, decoded by the documented layout (``DS_TILE`` in
  csrc/common.hpp: per tile slot, 1 KiB block (32-query group w, 32-key group
  kg, 16-query half t) at 8 w + 2 kg + t; the chunk of lane l -- key
  32 kg + l % 32, hi = l / 32 -- holds queries 32 w + 16 t + 4 hi + 8 j + i in
  slots 4 j + i and sits at position ds_pos(l, t) = l ^ (4 (l / 32) + 8 t);
  slot of row entry e of (b, h) = rep(b, h) * nnz + e), equal the fp64
  oracle's dS (``dense_probs_ds``) times one power of two per query tile, and
  are exactly zero at masked and padded elements -- a permuted or misplaced
  chunk fails this.
* End to end, both backward paths against the oracle under the parity gate,
  with dK and dV bitwise equal between them (the dK/dV kernel's arithmetic is
  the same with and without the stores).
"""
import ctypes
import math

import numpy as np
import pytest

from oracle import attention_oracle as ao
from tests.helpers import Floor, assert_close, oracle, seeded_inputs

torch = pytest.importorskip("torch")

pytestmark = pytest.mark.gpu


def _decode_index():
    """[128, 128] element offsets, inside one tile slot, of dS[q][k]."""
    q = np.arange(128)[:, None]
    k = np.arange(128)[None, :]
    w, t, qq = q // 32, (q % 32) // 16, q % 16
    kg, kl = k // 32, k % 32
    hi, j, i = (qq >> 2) & 1, qq >> 3, qq & 3
    lane = kl + 32 * hi
    pos = lane ^ (4 * (lane >> 5) + 8 * t)
    return (8 * w + 2 * kg + t) * 512 + pos * 8 + 4 * j + i


def _stored_ds(B, N, Hq, Hkv, d, dtype, seed, kw):
    """(stored dS as float64 [B, Hq, Npad, Lpad], oracle dS [B, Hq, N, L],
    allowed mask) after one mattn_bwd with MATTN_BWD_DS."""
    from jaxmodules_amd import _lib
    from jaxmodules_amd import attention as A

    lib = _lib.load()
    Q, K, V, dO = seeded_inputs(B, N, N, Hq, Hkv, d, seed)
    td = getattr(torch, dtype)
    q, k, v = (torch.from_numpy(x).to("cuda", td).contiguous() for x in (Q, K, V))
    do = torch.from_numpy(dO).to("cuda").contiguous()
    plan, tm = A.trace_call(tuple(q.shape), tuple(k.shape), tuple(v.shape), device=q.device, **kw)
    scale = 1.0 / math.sqrt(d)
    o, lse, res = A.mattn_forward(q, k, v, tm, scale, torch.float32, for_backward=True)
    dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
    p = A._problem(q, k, v, o, scale, do=do, dq=dq, dk=dk, dv=dv)
    bm = A.device_blockmap(tm, q.device)
    p.flags = _lib.MATTN_BWD_DS | _lib.MATTN_FWD_FOR_BWD
    base = int(lib.mattn_workspace_bytes(ctypes.byref(p)))
    total = int(lib.mattn_bwd_workspace_bytes(ctypes.byref(p), ctypes.byref(bm)))
    slots = tm.nnz * (B if tm.map_b == 1 else 1) * (Hq if tm.map_h == 1 else 1)
    assert total == base + slots * 128 * 128 * 2
    ws, wptr = A._workspace(total, q.device)
    _lib.check(lib.mattn_bwd(ctypes.byref(p), ctypes.byref(bm), q.data_ptr(), k.data_ptr(), v.data_ptr(),
                             o.data_ptr(), do.data_ptr(), lse.data_ptr(), A._aligned(res), wptr, total,
                             dq.data_ptr(), dk.data_ptr(), dv.data_ptr(), A._stream(q.device)), "mattn_bwd")
    torch.cuda.synchronize()
    off = wptr - ws.data_ptr() + base
    flat = ws[off:off + slots * 32768].view(torch.float16).double().cpu().numpy()
    idx = _decode_index()
    nqt, nkt = tm.nqt, tm.nkt
    got = np.full((B, Hq, nqt * 128, nkt * 128), np.nan)
    for b in range(B):
        for h in range(Hq):
            rep = (b if tm.map_b == 1 else 0) * (Hq if tm.map_h == 1 else 1) + (h if tm.map_h == 1 else 0)
            for qt in range(nqt):
                r = ((b % tm.map_b) * tm.map_h + h % tm.map_h) * nqt + qt
                for e in range(tm.row_ptr[r], tm.row_ptr[r + 1]):
                    kt = int(tm.row_ent[e, 0])
                    slot = rep * tm.nnz + e
                    got[b, h, qt * 128:(qt + 1) * 128, kt * 128:(kt + 1) * 128] = \
                        flat[slot * 16384 + idx]
    Qr, Kr, Vr = (x.float().cpu().numpy() for x in (q, k, v))
    allowed = oracle(Qr, Kr, Vr, dO, kw, grads=False)[3]
    _, ds = ao.dense_probs_ds(Qr, Kr, Vr, allowed, dO)
    return got, ds, allowed, tm


@pytest.mark.parametrize("case", [
    # (B, N, Hq, Hkv, d, dtype, seed, kw): broadcast causal map with GQA and
    # ragged tiles; a per-head map; a per-batch map with empty rows
    (2, 300, 4, 2, 128, "bfloat16", 3, dict(is_causal=True, block_size=128)),
    (1, 256, 4, 2, 128, "float16", 4, dict(mask_fn=lambda h, q, k: (q + 64 * h) >= k, block_size=128)),
    (2, 320, 2, 2, 128, "bfloat16", 5,
     dict(mask_fn=lambda b, h, q, k: ((q // (100 + 60 * b)) == (k // (100 + 60 * b))) & (q >= 128 * b),
          block_size=64)),
], ids=["causal_gqa_ragged", "per_head_map", "per_batch_map_empty_rows"])
def test_stored_fragments_are_ds_times_tile_power_of_two(case):
    B, N, Hq, Hkv, d, dtype, seed, kw = case
    print(f"[stored ds] fragments {case[:7]}", flush=True)
    got, ds, allowed, tm = _stored_ds(B, N, Hq, Hkv, d, dtype, seed, kw)
    nqt = tm.nqt
    present = ~np.isnan(got)
    for b in range(B):
        for h in range(Hq):
            for qt in range(nqt):
                rows = slice(qt * 128, min((qt + 1) * 128, N))
                g = got[b, h, rows, :N]
                r = ds[b, h, rows]
                m = allowed[b if allowed.shape[0] > 1 else 0, h if allowed.shape[1] > 1 else 0, rows]
                pres = present[b, h, rows, :N]
                assert np.all(pres[m]), "an allowed element lies in no stored tile"
                # masked elements of stored tiles, and the padding, are exactly zero
                assert np.all(g[pres & ~m] == 0)
                pad = got[b, h, qt * 128:(qt + 1) * 128][present[b, h, qt * 128:(qt + 1) * 128]]
                assert np.all(np.isfinite(pad))
                if not m.any():
                    continue
                c = float(np.sum(g[m] * r[m]) / max(np.sum(r[m] ** 2), 1e-300))
                e2 = round(math.log2(c))
                assert abs(math.log2(c) - e2) < 0.02, (b, h, qt, c)   # one power of two per tile
                err = np.abs(g[m] - 2.0 ** e2 * r[m]).max()
                assert err <= 1e-2 * 2.0 ** e2 * np.abs(r[m]).max(), (b, h, qt, err)


def _grads(shape, kw, dtype, store_ds, seed):
    import jaxmodules_amd as jm
    from jaxmodules_amd import attention as A

    B, N, L, Hq, Hkv, d = shape
    Q, K, V, dO = seeded_inputs(B, N, L, Hq, Hkv, d, seed)
    td = getattr(torch, dtype)
    q, k, v = (torch.from_numpy(x).to("cuda", td).requires_grad_() for x in (Q, K, V))
    old = A.STORE_DS
    A.STORE_DS = store_ds
    try:
        o = jm.masked_attention_via_map(q, k, v, **kw)
        o.backward(torch.from_numpy(dO).to("cuda"))
    finally:
        A.STORE_DS = old
    torch.cuda.synchronize()
    return (Q, K, V, dO, q, k, v), (q.grad, k.grad, v.grad)


END_TO_END = {
    "causal_gqa_ragged_bf16": ((2, 300, 300, 4, 2, 128), dict(is_causal=True, block_size=128), "bfloat16"),
    "partial_cross_fp16": ((1, 200, 330, 2, 1, 128),
                           dict(mask_fn=lambda h, q, k: (q + 3 * h - k) % 7 != 0, block_size=64), "float16"),
    "per_head_bf16": ((1, 256, 256, 4, 2, 128), dict(mask_fn=lambda h, q, k: (q + 64 * h) >= k,
                                                     block_size=128), "bfloat16"),
    "empty_query_tile_bf16": ((1, 384, 384, 2, 2, 128),
                              dict(mask_fn=lambda h, q, k: (q >= 128) & (q >= k), block_size=128), "bfloat16"),
    "head_dim_96_bf16": ((1, 200, 200, 2, 2, 96), dict(is_causal=True, block_size=64), "bfloat16"),
    "head_dim_64_forced_bf16": ((1, 256, 256, 2, 2, 64), dict(is_causal=True, block_size=128), "bfloat16"),
}


@pytest.mark.parametrize("name", list(END_TO_END))
def test_stored_ds_backward_matches_oracle_and_recompute(name):
    shape, kw, dtype = END_TO_END[name]
    print(f"[stored ds] end to end {name}", flush=True)
    inputs, g_ds = _grads(shape, kw, dtype, True, 21)
    _, g_rc = _grads(shape, kw, dtype, False, 21)
    assert torch.equal(g_ds[1], g_rc[1]), "dK differs between the stored-dS and recompute paths"
    assert torch.equal(g_ds[2], g_rc[2]), "dV differs between the stored-dS and recompute paths"
    if "empty" in name:
        assert torch.all(g_ds[0][:, :128] == 0)
    Q, K, V, dO, q, k, v = inputs
    Qr, Kr, Vr = (x.detach().float().cpu().numpy() for x in (q, k, v))
    _, _, g_ref, _ = oracle(Qr, Kr, Vr, dO, kw)
    floor = Floor()   # misses within the float16 operands' bound xfail (tests/helpers.py)
    for path, g in (("stored dS", g_ds), ("recompute", g_rc)):
        for nm, t, r in (("dQ", g[0], g_ref[0]), ("dK", g[1], g_ref[1]), ("dV", g[2], g_ref[2])):
            assert_close(t.float().cpu().numpy(), r, dtype, f"{name} {path} {nm}", floor=floor)
    floor.finish()
