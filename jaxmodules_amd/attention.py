"""Drop-in ``masked_attention_via_map`` running on the gfx950 HIP kernels.

Mirrors the public interface of ``/root/reference/jaxmodules/attention.py``:

* ``masked_attention_via_map(Q, K, V, *, is_causal, kernel_fn, mask_fn,
  block_size, window_size)`` -- same signature, argument meaning, exception
  types and output semantics as attention.py:347-455, with the reference's
  custom_vjp (attention.py:180,244-345) realised as a
  ``torch.autograd.Function`` whose forward calls ``mattn_fwd`` and whose
  backward calls ``mattn_bwd`` (the C ABI in ``include/mattn.h``);
* ``default_kernel`` / ``threshold_kernel`` (attention.py:18-50).

Arrays are torch tensors on the GPU (jax is not available in this image; the
jax.ffi binding a jax user would register is described with the C ABI).  The
layout is the reference's [B, L, H, d] (or [L, H, d]).  There is no CPU code
path: calling with the library unbuilt or with CPU tensors raises.
"""
from __future__ import annotations

import ctypes
import math
from collections import OrderedDict
from typing import Callable, Optional, Tuple

import numpy as np
import torch

from . import _lib
from . import blockmap as bmap

__all__ = ["masked_attention_via_map", "default_kernel", "threshold_kernel", "trace_call",
           "clear_cache", "mattn_forward", "mattn_backward"]


# ---------------------------------------------------------------------------
# kernel functions (attention.py:18-50)
# ---------------------------------------------------------------------------


def default_kernel(q, k):
    """exp(q . k / sqrt(d)) -- the reference's default score (attention.py:39-50).

    The kernels compute the same normalised weights as a softmax with scale
    1/sqrt(d) (the reference normalises by the running sum of this kernel)."""
    return np.exp(np.dot(q, k) / np.sqrt(np.shape(k)[-1]))


default_kernel._mattn_scale = None  # 1/sqrt(d)


def threshold_kernel(threshold: Optional[float] = None):
    """exp(q . k - threshold / sqrt(d)) (attention.py:18-36).

    The threshold term is a constant factor of every score and cancels in the
    normalisation, so this kernel is a softmax with scale 1."""

    def kernel_fn(q, k):
        dotp = np.dot(q, k)
        if threshold is not None:
            dotp = dotp - threshold / np.sqrt(np.shape(q)[0])
        return np.exp(dotp)

    kernel_fn._mattn_scale = 1.0
    return kernel_fn


def _kernel_scale(kernel_fn, d: int) -> float:
    s = getattr(kernel_fn, "_mattn_scale", "missing")
    if s == "missing":
        raise NotImplementedError(
            "only default_kernel and threshold_kernel are supported by the HIP kernels")
    return 1.0 / math.sqrt(d) if s is None else float(s)


# ---------------------------------------------------------------------------
# tile-map cache
# ---------------------------------------------------------------------------

_CACHE: "OrderedDict[tuple, bmap.TileMap]" = OrderedDict()
_CACHE_SIZE = 32


def clear_cache():
    _CACHE.clear()


def trace_call(q_shape, k_shape, v_shape, *, is_causal=False, mask_fn=None, block_size=None,
               window_size=None):
    """(Plan, TileMap) of a call; tile maps are cached per mask function and shapes
    (like the reference, which bakes mask_fn in at trace time under jax.jit)."""
    plan = bmap.make_plan(q_shape, k_shape, v_shape, is_causal=is_causal, mask_fn=mask_fn,
                          block_size=block_size, window_size=window_size)
    key = (bool(is_causal), mask_fn, block_size,
           None if window_size is None else tuple(window_size),
           plan.B, plan.N, plan.L, plan.Hq, plan.Hkv)
    tm = _CACHE.get(key)
    if tm is None:
        tm = bmap.trace(plan)
        _CACHE[key] = tm
        if len(_CACHE) > _CACHE_SIZE:
            _CACHE.popitem(last=False)
    else:
        _CACHE.move_to_end(key)
    return plan, tm


def device_blockmap(tm: bmap.TileMap, device) -> _lib.MattnBlockmap:
    """Uploads the tile map once per device and returns the C struct pointing at it."""
    key = str(torch.device(device))
    hit = tm.device.get(key)
    if hit is not None:
        return hit[1]

    def up(a):
        return torch.from_numpy(np.ascontiguousarray(a)).to(device)

    bufs = dict(
        row_ptr=up(tm.row_ptr), row_ent=up(tm.row_ent.reshape(-1)),
        col_ptr=up(tm.col_ptr), col_ent=up(tm.col_ent.reshape(-1)),
        row_bits=up(tm.row_bits.view(np.int64).reshape(-1)),
        col_bits=up(tm.col_bits.view(np.int64).reshape(-1)),
        q_order=up(tm.q_order), kv_order=up(tm.kv_order))
    s = _lib.MattnBlockmap(
        map_b=tm.map_b, map_h=tm.map_h, nqt=tm.nqt, nkt=tm.nkt, n_masks=tm.n_masks, nnz=tm.nnz,
        row_ptr=bufs["row_ptr"].data_ptr(), row_ent=bufs["row_ent"].data_ptr() if tm.nnz else None,
        col_ptr=bufs["col_ptr"].data_ptr(), col_ent=bufs["col_ent"].data_ptr() if tm.nnz else None,
        row_bits=bufs["row_bits"].data_ptr() if tm.n_masks else None,
        col_bits=bufs["col_bits"].data_ptr() if tm.n_masks else None,
        q_order=bufs["q_order"].data_ptr(), kv_order=bufs["kv_order"].data_ptr(),
        n_q_order=int(tm.q_order.size), n_kv_order=int(tm.kv_order.size))
    tm.device[key] = (bufs, s)
    return s


# ---------------------------------------------------------------------------
# C ABI calls
# ---------------------------------------------------------------------------

_DT = {torch.bfloat16: _lib.MATTN_BF16, torch.float16: _lib.MATTN_F16, torch.float32: _lib.MATTN_F32}


def _strides(t: torch.Tensor):
    s = t.stride()
    return (ctypes.c_int64 * 3)(s[0], s[1], s[2])


def _ready(t: torch.Tensor) -> torch.Tensor:
    """d contiguous and 16-byte aligned strides/base, as the kernels' vector loads need."""
    es = t.element_size()
    ok = t.stride(-1) == 1 and all((s * es) % 16 == 0 for s in t.stride()[:3]) \
        and t.data_ptr() % 16 == 0
    return t if ok else t.contiguous()


def _problem(q, k, v, o, scale, do=None, dq=None, dk=None, dv=None):
    B, N, Hq, d = q.shape
    p = _lib.MattnProblem(B=B, Lq=N, Lk=k.shape[1], Hq=Hq, Hkv=k.shape[2], D=d,
                          dtype=_DT[q.dtype], o_dtype=_DT[o.dtype], scale=scale)
    p.q_stride, p.k_stride, p.v_stride, p.o_stride = _strides(q), _strides(k), _strides(v), _strides(o)
    p.do_stride = _strides(do if do is not None else o)
    p.dq_stride = _strides(dq if dq is not None else q)
    p.dk_stride = _strides(dk if dk is not None else k)
    p.dv_stride = _strides(dv if dv is not None else v)
    return p


def _stream(device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def mattn_forward(q, k, v, tm: bmap.TileMap, scale: float, out_dtype=torch.float32):
    """O [B, N, Hq, d] (out_dtype) and base-2 LSE [B, Hq, N] via mattn_fwd."""
    lib = _lib.load()
    B, N, Hq, d = q.shape
    o = torch.empty((B, N, Hq, d), dtype=out_dtype, device=q.device)
    lse = torch.empty((B, Hq, N), dtype=torch.float32, device=q.device)
    p = _problem(q, k, v, o, scale)
    bm = device_blockmap(tm, q.device)
    _lib.check(lib.mattn_fwd(ctypes.byref(p), ctypes.byref(bm), q.data_ptr(), k.data_ptr(),
                             v.data_ptr(), o.data_ptr(), lse.data_ptr(), _stream(q.device)),
               "mattn_fwd")
    return o, lse


def mattn_backward(q, k, v, o, lse, do, tm: bmap.TileMap, scale: float):
    """(dQ, dK, dV) via mattn_bwd."""
    lib = _lib.load()
    dq = torch.empty_like(q)
    dk = torch.empty_like(k)
    dv = torch.empty_like(v)
    p = _problem(q, k, v, o, scale, do=do, dq=dq, dk=dk, dv=dv)
    ws = torch.empty(max(int(lib.mattn_workspace_bytes(ctypes.byref(p))), 256) + 256,
                     dtype=torch.uint8, device=q.device)
    wptr = (ws.data_ptr() + 255) & ~255
    bm = device_blockmap(tm, q.device)
    _lib.check(lib.mattn_bwd(ctypes.byref(p), ctypes.byref(bm), q.data_ptr(), k.data_ptr(),
                             v.data_ptr(), o.data_ptr(), do.data_ptr(), lse.data_ptr(), wptr,
                             dq.data_ptr(), dk.data_ptr(), dv.data_ptr(), _stream(q.device)),
               "mattn_bwd")
    return dq, dk, dv


class _MaskedAttention(torch.autograd.Function):
    """The reference's custom_vjp (attention.py:180, 244-345).  Residuals are
    (Q, K, V, O, LSE) instead of (Q, K, V): the backward reads the saved
    log-sum-exp rather than re-running the forward scan."""

    @staticmethod
    def forward(ctx, q, k, v, tm, scale, out_dtype):
        o, lse = mattn_forward(q, k, v, tm, scale, out_dtype)
        ctx.save_for_backward(q, k, v, o, lse)
        ctx.tm, ctx.scale = tm, scale
        return o

    @staticmethod
    def backward(ctx, do):
        q, k, v, o, lse = ctx.saved_tensors
        do = _ready(do.to(o.dtype))
        dq, dk, dv = mattn_backward(q, k, v, o, lse, do, ctx.tm, ctx.scale)
        return dq, dk, dv, None, None, None


def masked_attention_via_map(
    Q: torch.Tensor,
    K: torch.Tensor,
    V: torch.Tensor,
    *,
    is_causal: bool = False,
    kernel_fn: Callable = default_kernel,
    mask_fn: Optional[Callable] = None,
    block_size: Optional[int] = None,
    window_size: Optional[Tuple[int, int]] = None,
    out_dtype: Optional[torch.dtype] = None,
) -> torch.Tensor:
    """Memory-efficient masked attention (attention.py:347-455).

    K: [B, L, Hkv, d] or [L, Hkv, d]; Q: [B, N, Hq, d] or [N, Hq, d]; V like K.
    is_causal: mask q >= k (exclusive with mask_fn, ValueError otherwise).
    kernel_fn: default_kernel (softmax with scale 1/sqrt(d)) or threshold_kernel(t)
        (scale 1); other kernels raise NotImplementedError.
    mask_fn: boolean function of (b, h, q, k) or (h, q, k), elementwise in its
        index arguments (it is evaluated on broadcast numpy index arrays).
    block_size / window_size: as the reference: the window is block-granular,
        clamped at the sequence edges, and may change results (attention.py:374-381).
    out_dtype: dtype of the output.  Default float32, which is what the
        reference returns (its running accumulators are float32,
        attention.py:173); pass Q.dtype for a 16-bit output.

    Returns [B, N, Hq, d] (or [N, Hq, d]); differentiable w.r.t. Q, K, V.
    Rows with no allowed key are zero (attention.py:91-100).
    """
    plan, tm = trace_call(tuple(Q.shape), tuple(K.shape), tuple(V.shape), is_causal=is_causal,
                          mask_fn=mask_fn, block_size=block_size, window_size=window_size)
    scale = _kernel_scale(kernel_fn, plan.d)
    if not (Q.is_cuda and K.is_cuda and V.is_cuda):
        raise RuntimeError("masked_attention_via_map runs on the GPU only (no CPU code path)")
    dt = torch.promote_types(torch.promote_types(Q.dtype, K.dtype), V.dtype)
    if dt not in _DT:
        raise TypeError(f"unsupported dtype {dt}")
    if plan.squeeze_batch:
        Q, K, V = Q[None], K[None], V[None]
    q, k, v = (_ready(x.to(dt)) for x in (Q, K, V))
    od = torch.float32 if out_dtype is None else out_dtype
    if dt == torch.float32 and od != torch.float32:
        raise TypeError("float32 inputs produce a float32 output")
    if od not in (torch.float32, dt):
        raise TypeError(f"out_dtype must be float32 or {dt}")
    out = _MaskedAttention.apply(q, k, v, tm, scale, od)
    return out[0] if plan.squeeze_batch else out
