"""Parity at the BASELINE configurations' full sizes (GPU).

The fp64 CPU oracle cannot run at these sizes, so for a floating-point kernel
the check is a float32 torch reference on the GPU (dense masked softmax
attention, chunked over queries, every key) for sampled heads, under the same
element-wise gate as the oracle tests (2e-3 + 2e-3 |b| + half an ulp of the
output dtype).  Every head is further checked through two identities that hold
for any input, whatever the size:
  * sum_k dV[b, k, hk] = sum over the group's heads h and non-empty rows q of dO[b, q, h]
    (the attention weights of a row sum to one);
  * sum_k dK[b, k, hk] = 0  (sum_k dS[q, k] = 0 for every row).
"""
import math

import numpy as np
import pytest

from tests.helpers import assert_close

torch = pytest.importorskip("torch")

pytestmark = pytest.mark.gpu


def _docs(L, seed, mean=2048, minlen=64):
    rng = np.random.default_rng(seed)
    lens = []
    while sum(lens) < L:
        lens.append(max(minlen, int(rng.geometric(1.0 / mean))))
    return np.repeat(np.arange(len(lens)), lens)[:L]


def config(name):
    """(B, L, H, d, kwargs, numpy mask of (h, q[:,None], k[None,:]) for the sampled heads)."""
    if name == "cfg2":
        kw = dict(is_causal=True, block_size=128)
        return 4, 4096, 32, 128, kw, lambda h, q, k: q >= k
    if name == "target":   # the north star's shape
        kw = dict(is_causal=True, block_size=128)
        return 1, 8192, 32, 128, kw, lambda h, q, k: q >= k
    if name == "cfg3":
        m = lambda b, h, q, k: (q >= k) & (q - k <= 512)
        kw = dict(mask_fn=m, window_size=(512, 0), block_size=128)
        return 2, 16384, 16, 128, kw, lambda h, q, k: (q >= k) & (q - k <= 512)
    if name == "cfg4":
        nt, H = 64, 32
        rng = np.random.default_rng(4)
        tbl = rng.random((H, nt, nt)) < 0.25
        tbl[:, np.arange(nt), np.arange(nt)] = True
        m = lambda b, h, q, k: tbl[h, q // 128, k // 128] & ((q // 128 != k // 128) | (q >= k))
        return 1, 8192, H, 64, dict(mask_fn=m, block_size=128), \
            lambda h, q, k: tbl[h, q // 128, k // 128] & ((q // 128 != k // 128) | (q >= k))
    if name == "cfg5":
        doc = _docs(32768, 5)
        m = lambda b, h, q, k: (doc[q] == doc[k]) & (q >= k)
        return 1, 32768, 8, 128, dict(mask_fn=m, block_size=128), \
            lambda h, q, k: (doc[q] == doc[k]) & (q >= k)
    raise KeyError(name)


def reference_head(q, k, v, do, allowed_fn, h, chunk):
    """float32 dense reference for one (b, h): O, dQ, dK, dV; q/k/v/do [L, d] float32."""
    L, d = q.shape
    scale = 1.0 / math.sqrt(d)
    kidx = np.arange(L)
    O = torch.empty_like(q)
    dQ = torch.empty_like(q)
    dK = torch.zeros_like(k)
    dV = torch.zeros_like(v)
    for q0 in range(0, L, chunk):
        qi = np.arange(q0, min(L, q0 + chunk))
        allowed = torch.from_numpy(np.asarray(allowed_fn(h, qi[:, None], kidx[None, :]), bool)).to(q.device)
        s = (q[q0:q0 + len(qi)] @ k.T) * scale
        s = s.masked_fill(~allowed, float("-inf"))
        m = s.amax(dim=1, keepdim=True)
        m = torch.where(torch.isfinite(m), m, torch.zeros_like(m))
        p = torch.exp(s - m).masked_fill(~allowed, 0.0)
        den = p.sum(dim=1, keepdim=True)
        p = p / torch.where(den > 0, den, torch.ones_like(den))
        g = do[q0:q0 + len(qi)]
        O[q0:q0 + len(qi)] = p @ v
        dp = g @ v.T
        delta = (dp * p).sum(dim=1, keepdim=True)
        ds = p * (dp - delta)
        dQ[q0:q0 + len(qi)] = (ds @ k) * scale
        dK += (ds.T @ q[q0:q0 + len(qi)]) * scale
        dV += p.T @ g
    return O, dQ, dK, dV


@pytest.mark.parametrize("name", ["cfg2", "cfg3", "cfg4", "cfg5", "target"])
def test_baseline_config_full_size(name):
    import jaxmodules_amd as jm

    print(f"[fullsize] {name}", flush=True)
    B, L, H, d, kw, allowed_fn = config(name)
    dev = torch.device("cuda")
    g = torch.Generator(device=dev)
    g.manual_seed(1234)
    f = d ** -0.25
    q = (torch.randn((B, L, H, d), generator=g, device=dev) * f).to(torch.bfloat16).requires_grad_()
    k = (torch.randn((B, L, H, d), generator=g, device=dev) * f).to(torch.bfloat16).requires_grad_()
    v = (torch.randn((B, L, H, d), generator=g, device=dev) * f).to(torch.bfloat16).requires_grad_()
    do = torch.randn((B, L, H, d), generator=g, device=dev)
    o = jm.masked_attention_via_map(q, k, v, **kw)
    o.backward(do)
    torch.cuda.synchronize()
    assert o.dtype == torch.float32 and q.grad.dtype == torch.bfloat16

    # sampled heads against the float32 reference
    chunk = max(256, (1 << 27) // L)
    for b, h in ((0, 0), (B - 1, H - 1)):
        with torch.no_grad():
            ref = reference_head(q[b, :, h].detach().float(), k[b, :, h].detach().float(),
                                 v[b, :, h].detach().float(), do[b, :, h], allowed_fn, h, chunk)
        got = (o[b, :, h], q.grad[b, :, h], k.grad[b, :, h], v.grad[b, :, h])
        for what, x, r in zip(("O", "dQ", "dK", "dV"), got, ref):
            out_name = "float32" if what == "O" else "bfloat16"
            assert_close(x.detach().float().cpu().numpy(), r.cpu().numpy(), "bfloat16",
                         f"{name} b={b} h={h} {what}", out_name)

    # identities over every head (GQA group = 1 here; every configuration allows
    # the diagonal, so no row is empty)
    sum_dv = v.grad.float().sum(dim=1)                     # [B, H, d]
    sum_do = do.sum(dim=1)
    scale_ = do.abs().sum(dim=1).clamp_min(1.0)
    rel = ((sum_dv - sum_do).abs() / scale_).max().item()
    sum_dk = k.grad.float().sum(dim=1)
    scale_k = k.grad.float().abs().sum(dim=1).clamp_min(1e-6)
    relk = (sum_dk.abs() / scale_k).max().item()
    print(f"[fullsize] {name}: identity deviations dV {rel:.3g}, dK {relk:.3g}", flush=True)
    assert rel < 5e-4, f"{name}: sum_k dV vs sum_q dO, max relative deviation {rel:.3g}"
    assert relk < 5e-3, f"{name}: sum_k dK should vanish, max relative {relk:.3g}"
