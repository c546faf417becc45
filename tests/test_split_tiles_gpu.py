"""Split tiles (GPU): the forward's per-query-tile largest attention weight
(``pmx`` in the residual), which decides the 128-row query tiles whose
forward and backward run again with their float16 operands' rounded-off
parts (the rows with a dominant key, where float16 P, dS and dO would leave a
bfloat16 gradient one ulp past the parity gate).

* pmx, read from the residual at its documented place (after the float16 V'
  and Q' copies, the V' scales and maxima and the Q' scales, each block
  256-byte aligned), equals the oracle's largest softmax weight over each
  tile's rows (to float16 rounding of the forward's normaliser), and the
  split-row mask after it flags exactly the rows whose largest weight reaches
  SPLIT_P, for causal, document and unit-variance problems, and the flag per
  key tile after that (set by the split rows' walk of the forward) marks
  exactly the dK/dV columns where a split row of the kv head's query heads
  has an allowed key;
* the split-tile problems these masks make (a quarter to all of the tiles
  split) meet the parity gate in every output, with a float32 and a bfloat16
  output, without the float16-floor allowance, at d = 64 (split passes inside
  the main kernels) and d = 128 (separate split kernels).
"""
import math

import numpy as np
import pytest

from tests.helpers import assert_close, oracle, seeded_inputs

torch = pytest.importorskip("torch")

pytestmark = pytest.mark.gpu

SPLIT_P = 1 / 32  # common.hpp SPLIT_P


def _align(x):
    return (x + 255) // 256 * 256


def _pmx(res, B, Hq, Hkv, N, L, D):
    """The residual's [B, Hq, nqt] per-tile largest weights, [B, Hq, nqt * 128]
    split-row flags (the 128-bit mask per tile that follows them) and
    [B, Hkv, nkt] split-column flags (one int per key tile after those)."""
    nqt, nkt = -(-N // 128), -(-L // 128)
    qt, kt = B * Hq * nqt, B * Hkv * nkt
    off = _align(kt * 128 * D * 2) + _align(qt * 128 * D * 2) + 2 * _align(kt * 4) + _align(qt * 4)
    base = (res.data_ptr() + 255) // 256 * 256 - res.data_ptr()
    pmx = res[base + off:base + off + qt * 4].view(torch.float32).cpu().numpy().reshape(B, Hq, nqt)
    off += _align(qt * 4)
    words = res[base + off:base + off + qt * 16].view(torch.int32).cpu().numpy().astype(np.uint32)
    bits = (words.reshape(qt, 4)[:, :, None] >> np.arange(32, dtype=np.uint32)) & 1
    off += _align(qt * 16)
    scol = res[base + off:base + off + kt * 4].view(torch.int32).cpu().numpy().reshape(B, Hkv, nkt)
    return pmx, bits.reshape(B, Hq, nqt * 128).astype(bool), scol != 0


def _masks():
    from jaxmodules_amd import masks

    doc = np.repeat(np.arange(40), np.random.default_rng(7).integers(1, 60, size=40))[:300]
    return {
        "causal": dict(is_causal=True),
        "documents": dict(mask_fn=masks.intersect(masks.documents(doc), masks.causal())),
        "window": dict(mask_fn=lambda b, h, q, k: (k <= q) & (q - k <= 40), block_size=64),
    }


@pytest.mark.parametrize("d", [64, 128])
@pytest.mark.parametrize("scaled", [True, False], ids=["scaled", "unit"])
@pytest.mark.parametrize("mask", ["causal", "documents", "window"])
def test_pmx_is_each_query_tiles_largest_weight(mask, scaled, d):
    from jaxmodules_amd import attention as A

    B, N, Hq, Hkv = 2, 300, 4, 2
    kw = _masks()[mask]
    print(f"[split] pmx mask={mask} scaled={scaled} d={d}", flush=True)
    Q, K, V, _ = seeded_inputs(B, N, N, Hq, Hkv, d, 97, scaled=scaled)
    q, k, v = (torch.from_numpy(x).to("cuda", torch.bfloat16) for x in (Q, K, V))
    plan, tm = A.trace_call(tuple(q.shape), tuple(k.shape), tuple(v.shape), device=q.device, **kw)
    o, lse, res = A.mattn_forward(q, k, v, tm, 1 / math.sqrt(d), torch.float32, for_backward=True)
    torch.cuda.synchronize()
    got, split, scol = _pmx(res, B, Hq, Hkv, N, N, d)
    # the oracle's weights on the same (rounded) inputs
    Qr, Kr, Vr = (x.float().cpu().numpy().astype(np.float64) for x in (q, k, v))
    _, _, _, allowed = oracle(Qr, Kr, Vr, None, kw, grads=False)
    S = np.einsum("bqhd,bkhd->bhqk", Qr, np.repeat(Kr, Hq // Hkv, axis=2)) / math.sqrt(d)
    S = np.where(allowed, S, -np.inf)
    m = S.max(-1, keepdims=True)
    P = np.where(allowed, np.exp(S - np.where(np.isfinite(m), m, 0)), 0)
    den = P.sum(-1, keepdims=True)
    P = P / np.where(den > 0, den, 1)
    nqt = got.shape[-1]
    pm = np.zeros((B, Hq, nqt * 128))
    pm[..., :P.shape[2]] = P.max(-1)
    want = pm.reshape(B, Hq, nqt, 128).max(-1)
    np.testing.assert_allclose(got, want, rtol=2e-3, atol=1e-7)
    # the split rows: largest weight at least SPLIT_P (rows within rounding of it excepted)
    rowmax = P.max(-1)
    clear = np.abs(rowmax / SPLIT_P - 1) > 2e-3
    assert np.array_equal(split[..., :N][clear], (rowmax >= SPLIT_P)[clear])
    # a tile with a split row has its largest weight at least SPLIT_P
    nq = split.shape[-1] // 128
    assert np.array_equal(split.reshape(B, Hq, nq, 128).any(-1), got >= SPLIT_P)
    # the split columns: key tiles where a split row of a query head of the kv
    # head's group has an allowed key
    nkt = scol.shape[-1]
    reach = np.zeros((B, Hq, nkt * 128), bool)
    reach[..., :N] = (np.broadcast_to(allowed, (B, Hq, N, N)) & split[..., :N, None]).any(2)
    want_col = reach.reshape(B, Hkv, Hq // Hkv, nkt, 128).any((2, 4))
    assert np.array_equal(scol, want_col), (scol.sum(), want_col.sum())
    frac = (want >= SPLIT_P).mean()
    print(f"[split] {mask} scaled={scaled}: {frac:.2f} of the tiles split, "
          f"{want_col.mean():.2f} of the columns", flush=True)
    assert frac > 0  # every one of these masks has rows with a dominant key


@pytest.mark.parametrize("d", [64, 128])
@pytest.mark.parametrize("out", [None, "bfloat16"], ids=["out_f32", "out_bf16"])
@pytest.mark.parametrize("mask", ["causal", "documents", "window"])
def test_split_tile_problems_meet_the_gate(mask, out, d):
    """Unit-variance bfloat16 inputs, where many tiles are split: every output
    within the gate, no float16-floor allowance."""
    import jaxmodules_amd as jm

    B, N, Hq, Hkv = 2, 300, 4, 2
    kw = _masks()[mask]
    print(f"[split] gate mask={mask} out={out} d={d}", flush=True)
    Q, K, V, dO = seeded_inputs(B, N, N, Hq, Hkv, d, 101, scaled=False)
    q, k, v = (torch.from_numpy(x).to("cuda", torch.bfloat16).requires_grad_() for x in (Q, K, V))
    od = None if out is None else torch.bfloat16
    o = jm.masked_attention_via_map(q, k, v, out_dtype=od, **kw)
    do_t = torch.from_numpy(dO).to("cuda", o.dtype)
    Qr, Kr, Vr = (x.detach().float().cpu().numpy() for x in (q, k, v))
    O_ref, _, g_ref, _ = oracle(Qr, Kr, Vr, do_t.float().cpu().numpy(), kw)
    out_name = "float32" if out is None else out
    assert_close(o.detach().float().cpu().numpy(), O_ref, "bfloat16", "O", out_name)
    o.backward(do_t)
    for name, t, r in (("dQ", q, g_ref[0]), ("dK", k, g_ref[1]), ("dV", v, g_ref[2])):
        assert_close(t.grad.float().cpu().numpy(), r, "bfloat16", name)
    torch.cuda.synchronize()
