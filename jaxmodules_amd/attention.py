"""Drop-in ``masked_attention_via_map`` running on the gfx950 HIP kernels.

Mirrors the public interface of ``/root/reference/jaxmodules/attention.py``:

* ``masked_attention_via_map(Q, K, V, *, is_causal, kernel_fn, mask_fn,
  block_size, window_size)`` -- same signature, argument meaning, exception
  types and output semantics as attention.py:347-455, with the reference's
  custom_vjp (attention.py:180,244-345) realised as a
  ``torch.autograd.Function`` whose forward calls ``mattn_fwd`` and whose
  backward calls ``mattn_bwd`` (the C ABI in ``include/mattn.h``);
* ``default_kernel`` / ``threshold_kernel`` (attention.py:18-50);
* ``flex_attention(query, key, value, score_mod, block_mask, scale,
  enable_gqa, return_lse)`` (attention.py:456-692) on the same kernels, its
  ``BlockMask`` handed over as a tile map (``BlockMask.tile_map``).

The kernels are built for head dimensions 64, 128 and 256; other head
dimensions up to 256 are zero-padded on the GPU to the next of the three (zero
columns of Q and K leave every score unchanged, zero columns of V give zero
output columns, which are sliced off; the scale stays 1/sqrt(true d)).  16-bit
inputs at 64 and 128 run on the MFMA kernels; float32 inputs, and every dtype
at 256, on float32 SIMT kernels.

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

__all__ = ["masked_attention_via_map", "flex_attention", "flex_attention_slow", "default_kernel",
           "threshold_kernel", "use_custom_einsum", "kernel_scale", "trace_call", "clear_cache",
           "mattn_forward", "mattn_backward"]


def use_custom_einsum():
    """attention.py:12-15: the reference switches its P.V contraction to the
    vmap-based einsum of vectorize.py:264-382 for precision (its own tests call
    this first).  Here P.V is a float16 MFMA product accumulated in float32, so
    there is nothing to switch; kept so that such code imports and runs."""
    return None


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


_PROBED: "OrderedDict[tuple, float]" = OrderedDict()  # bounded like the tile-map cache


def _call_kernel(kernel_fn, q, k) -> float:
    """kernel_fn on 1-D float64 vectors: numpy arrays first, torch tensors if the
    function cannot take those (the reference's kernels use jnp.dot / jnp.exp)."""
    try:
        return float(kernel_fn(q, k))
    except Exception:
        return float(kernel_fn(torch.from_numpy(q), torch.from_numpy(k)))


def kernel_scale(kernel_fn, d: int) -> float:
    """The softmax scale s of a kernel_fn(q, k) = exp(s * q.k + c).

    The reference normalises the kernel's scores over each row's allowed keys
    (attention.py:83-100), so a constant factor exp(c) cancels and every such
    kernel is a softmax with scale s: default_kernel has s = 1/sqrt(d),
    threshold_kernel(t) s = 1 (attention.py:18-50), and a user kernel such as
    the reference test's exp(q.k / (2 sqrt(d))) (test_mapped_attention.py:1122-1144)
    s = 1/(2 sqrt(d)).  Other kernels are probed: log kernel_fn(q, k) on 12
    seeded random pairs of length d must be an affine function of q.k (relative
    residual <= 1e-5), else NotImplementedError, since a kernel of any other form
    has no counterpart in the HIP kernels.  s may be negative or zero (the caller
    folds the sign into Q)."""
    s = getattr(kernel_fn, "_mattn_scale", "missing")
    if s != "missing":
        return 1.0 / math.sqrt(d) if s is None else float(s)
    key = (_mask_key(kernel_fn), d)  # by content, like mask functions (identity as fallback)
    if key in _PROBED:
        _PROBED.move_to_end(key)
        return _PROBED[key]
    rng = np.random.default_rng(1234)
    xs, ys = [], []
    for _ in range(12):
        q = rng.standard_normal(d) * d ** -0.25
        k = rng.standard_normal(d) * d ** -0.25
        try:
            val = _call_kernel(kernel_fn, q, k)
        except Exception as e:
            raise NotImplementedError(f"kernel_fn could not be evaluated on vectors of length {d}: {e}")
        if not (val > 0 and math.isfinite(val)):
            raise NotImplementedError("kernel_fn must be exp(s * q.k + c) (positive, finite scores)")
        xs.append(float(np.dot(q, k)))
        ys.append(math.log(val))
    A = np.stack([np.array(xs), np.ones(len(xs))], 1)
    (sc, c), *_ = np.linalg.lstsq(A, np.array(ys), rcond=None)
    resid = np.abs(A @ np.array([sc, c]) - np.array(ys))
    if resid.max() > 1e-5 * (1.0 + np.abs(ys).max()):
        raise NotImplementedError(
            "only kernels of the form exp(s * q.k + c) are supported by the HIP kernels "
            f"(log kernel_fn is not affine in q.k: residual {resid.max():.3g})")
    # snap to the nearest float32 value: the probe sees float32 arithmetic in
    # jnp-based kernels, while the scale itself is a float32 kernel argument
    sc = float(np.float32(sc))
    _PROBED[key] = sc
    if len(_PROBED) > _CACHE_SIZE:
        _PROBED.popitem(last=False)
    return sc


# ---------------------------------------------------------------------------
# tile-map cache
# ---------------------------------------------------------------------------

_CACHE: "OrderedDict[tuple, bmap.TileMap]" = OrderedDict()
_CACHE_SIZE = 32


class _Unfrozen(Exception):
    pass


# modules whose functions and classes are keyed by name: their behaviour is
# fixed by the installed library, not by values a caller can change
_LIB_MODULES = ("numpy", "torch", "math", "builtins", "operator")


def _lib_object(v) -> bool:
    mod = getattr(v, "__module__", None) or type(v).__module__ or ""
    return mod.split(".")[0] in _LIB_MODULES


def _freeze(v, depth=0, names=()):
    """A hashable value standing for what ``v`` contributes to a mask function's
    result: plain values as they are, containers and numpy arrays (and small
    host tensors) by content, functions by their own key, library functions and
    classes by name, and a module by the values of those of its attributes that
    the mask's code names (``names``: its co_names, which hold every global
    and attribute it reads), so that a changed module attribute gives another
    key; anything else raises _Unfrozen."""
    import types

    if depth > 8:
        raise _Unfrozen
    if v is None or isinstance(v, (bool, int, float, complex, str, bytes)):
        return (type(v).__name__, v)
    if isinstance(v, np.generic):
        return ("np", v.dtype.str, v.item())
    if isinstance(v, np.ndarray):
        import hashlib
        return ("nd", v.dtype.str, v.shape, hashlib.sha1(np.ascontiguousarray(v).tobytes()).hexdigest())
    if isinstance(v, torch.Tensor):
        if v.is_cuda or v.numel() > (1 << 24):
            raise _Unfrozen
        return _freeze(v.detach().numpy(), depth + 1)
    if isinstance(v, (tuple, list, frozenset, set)):
        items = sorted(v, key=repr) if isinstance(v, (set, frozenset)) else v
        return (type(v).__name__, tuple(_freeze(x, depth + 1, names) for x in items))
    if isinstance(v, dict):
        return ("dict", tuple(sorted(((repr(k), _freeze(x, depth + 1, names)) for k, x in v.items()))))
    if isinstance(v, types.ModuleType):
        d = vars(v)
        return ("module", v.__name__, tuple((n, _freeze(d[n], depth + 1, names)) for n in sorted(names) if n in d))
    if isinstance(v, types.FunctionType):
        return ("fn", _fn_content(v, depth + 1))
    if isinstance(v, (types.BuiltinFunctionType, np.ufunc)) or (
            (isinstance(v, type) or type(v).__name__ == "_ArrayFunctionDispatcher") and _lib_object(v)):
        return ("builtin", getattr(v, "__module__", None), getattr(v, "__qualname__", None),
                getattr(v, "__name__", None))
    raise _Unfrozen


def _fn_content(fn, depth=0):
    """What a plain Python function computes, as a hashable value: its code,
    defaults, closure contents and the values of the globals its code names
    (read now, so a changed value gives another key)."""
    code = fn.__code__
    names, stack = set(), [code]
    while stack:  # the names of nested code objects (inner lambdas) too
        c = stack.pop()
        names.update(c.co_names)
        stack.extend(x for x in c.co_consts if hasattr(x, "co_names"))
    g = fn.__globals__
    try:
        cells = tuple(_freeze(c.cell_contents, depth + 1, names) for c in (fn.__closure__ or ()))
    except ValueError:  # an empty closure cell
        raise _Unfrozen
    return (code, _freeze(fn.__defaults__, depth + 1, names), _freeze(fn.__kwdefaults__, depth + 1, names), cells,
            tuple((n, _freeze(g[n], depth + 1, names)) for n in sorted(names) if n in g))


def _mask_key(mask_fn):
    """Cache key of a mask function: by content when every value it reads is
    one _freeze can describe -- so a new but identical lambda per call (the
    usual way to pass a mask) finds the map already traced -- and the function
    object itself otherwise."""
    import types

    if isinstance(mask_fn, types.FunctionType):
        try:
            return ("content", _fn_content(mask_fn))
        except (_Unfrozen, TypeError, RecursionError):
            pass
    return mask_fn


def clear_cache():
    _CACHE.clear()
    _BM_CACHE.clear()


def trace_call(q_shape, k_shape, v_shape, *, is_causal=False, mask_fn=None, block_size=None,
               window_size=None, device=None):
    """(Plan, TileMap) of a call; tile maps are cached per mask function and shapes
    (like the reference, which bakes mask_fn in at trace time under jax.jit).

    With a GPU ``device``, masks in closed form (``jaxmodules_amd.masks``,
    ``is_causal`` and no mask) are classified on that GPU
    (``blockmap.device_trace``); other mask functions are traced on the host.
    Both give the same map."""
    plan = bmap.make_plan(q_shape, k_shape, v_shape, is_causal=is_causal, mask_fn=mask_fn,
                          block_size=block_size, window_size=window_size)
    key = (bool(is_causal), _mask_key(mask_fn), block_size,
           None if window_size is None else tuple(window_size),
           plan.B, plan.N, plan.L, plan.Hq, plan.Hkv)
    tm = _CACHE.get(key)
    if tm is None:
        on_gpu = device is not None and torch.device(device).type == "cuda"
        if on_gpu and bmap.spec_of(plan.mask4) is not None:
            tm = bmap.device_trace(plan, device)
        else:
            tm = bmap.trace(plan)
        _CACHE[key] = tm
        if len(_CACHE) > _CACHE_SIZE:
            _CACHE.popitem(last=False)
    else:
        _CACHE.move_to_end(key)
    return plan, tm


def _check_map(tm: bmap.TileMap, q, k):
    """The tile map must be traced for this problem's shape: its launch orders
    enumerate (b, head, tile) items of exactly these sizes."""
    B, N, Hq, _ = q.shape
    got = (tm.B, tm.Lq, tm.Hq, tm.Lk, tm.Hkv)
    want = (B, N, Hq, k.shape[1], k.shape[2])
    if got != want:
        raise ValueError(f"tile map traced for (B, Lq, Hq, Lk, Hkv) = {got}, called with {want}")


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
        col_ptr=up(tm.col_ptr), col_ent=up(tm.col_ent.reshape(-1)), col_row=up(tm.col_row),
        kv_desc=up(tm.kv_desc.reshape(-1)),
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
        n_q_order=int(tm.q_order.size), n_kv_order=int(tm.kv_order.size),
        col_row=bufs["col_row"].data_ptr() if tm.nnz else None, kv_desc=bufs["kv_desc"].data_ptr())
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


def mattn_forward(q, k, v, tm: bmap.TileMap, scale: float, out_dtype=torch.float32,
                  heads_major: bool = False, for_backward: bool = False, precise: bool = False):
    """(O [B, N, Hq, d] in out_dtype, base-2 LSE [B, Hq, N], residual) via
    mattn_fwd.  ``heads_major`` lays O out in memory as [B, Hq, N, d] (the
    returned tensor is the [B, N, Hq, d] view of it).  The residual (a uint8
    tensor; None for float32 inputs, at d = 256 and with ``precise``, which
    the SIMT kernels serve) holds the float16 V copy and, with
    ``for_backward``, the float16 Q copy that mattn_backward reads.
    ``precise``: float32 arithmetic for 16-bit inputs (MATTN_PRECISE)."""
    lib = _lib.load()
    B, N, Hq, d = q.shape
    if heads_major:
        o = torch.empty((B, Hq, N, d), dtype=out_dtype, device=q.device).transpose(1, 2)
    else:
        # q's memory order when q is a dense view (the residue rewrite's strided
        # [P, L / P, H, d] view), so that O lands in the caller's order
        o = torch.empty_like(q, dtype=out_dtype)
    lse = torch.empty((B, Hq, N), dtype=torch.float32, device=q.device)
    _check_map(tm, q, k)
    p = _problem(q, k, v, o, scale)
    p.flags = (_lib.MATTN_FWD_FOR_BWD if for_backward else 0) | (_lib.MATTN_PRECISE if precise else 0)
    bm = device_blockmap(tm, q.device)
    nws = int(lib.mattn_fwd_workspace_bytes(ctypes.byref(p)))
    res, rptr = _workspace(nws, q.device)
    _lib.check(lib.mattn_fwd(ctypes.byref(p), ctypes.byref(bm), q.data_ptr(), k.data_ptr(),
                             v.data_ptr(), o.data_ptr(), lse.data_ptr(), rptr, _stream(q.device)),
               "mattn_fwd")
    return o, lse, res


def _workspace(nbytes: int, device):
    """(tensor, 256-byte aligned pointer) of at least nbytes of device memory
    (None, None when nbytes is 0)."""
    if nbytes == 0:
        return None, None
    ws = torch.empty(nbytes + 256, dtype=torch.uint8, device=device)
    return ws, _aligned(ws)


def _aligned(t):
    return None if t is None else (t.data_ptr() + 255) & ~255


# Whether the backward keeps dS (MATTN_BWD_DS): None = where it pays and fits
# (16-bit inputs at kernel head dim 128, the dS workspace at most DS_MAX_BYTES),
# True = wherever the kernels support it (16-bit inputs, head dim <= 128),
# False = never.  The stored dS takes 2 bytes per pair of every present tile,
# O(L^2 density) -- 2.2 GB at B=1 L=8192 H=32 causal, 8.7 GB at L=16384 --
# where the recomputing backward needs O(L) workspace like the reference
# (attention.py:233-237 keeps memory at O(block_size L)).  By default its extra
# workspace is therefore bounded by DS_MAX_BYTES, 4 GiB (1.5% of an MI355X's
# 288 GB); larger problems recompute dS in the dQ pass (4 D flop per pair).
STORE_DS: Optional[bool] = None
DS_MAX_BYTES = 4 << 30


def bwd_flags(p, bm) -> int:
    """mattn_problem.flags for the backward of problem ``p`` on map ``bm``: the
    forward's flags plus MATTN_BWD_DS where STORE_DS selects it."""
    lib = _lib.load()
    flags = p.flags & ~_lib.MATTN_BWD_DS
    if STORE_DS is False or p.dtype == _lib.MATTN_F32 or p.D > 128 or (p.flags & _lib.MATTN_PRECISE):
        return flags
    if STORE_DS is None:
        if p.D != 128:
            return flags
        p.flags = flags | _lib.MATTN_BWD_DS
        extra = int(lib.mattn_bwd_workspace_bytes(ctypes.byref(p), ctypes.byref(bm))) \
            - int(lib.mattn_workspace_bytes(ctypes.byref(p)))
        p.flags = flags
        if extra > DS_MAX_BYTES:
            return flags
    return flags | _lib.MATTN_BWD_DS


def mattn_backward(q, k, v, o, lse, do, tm: bmap.TileMap, scale: float, res=None, precise: bool = False):
    """(dQ, dK, dV) via mattn_bwd; ``res`` is mattn_forward's residual (run
    with for_backward=True and the same ``precise``)."""
    lib = _lib.load()
    _check_map(tm, q, k)
    dq = torch.empty_like(q)
    dk = torch.empty_like(k)
    dv = torch.empty_like(v)
    p = _problem(q, k, v, o, scale, do=do, dq=dq, dk=dk, dv=dv)
    p.flags = _lib.MATTN_FWD_FOR_BWD | (_lib.MATTN_PRECISE if precise else 0)
    bm = device_blockmap(tm, q.device)
    p.flags = bwd_flags(p, bm)
    nws = int(lib.mattn_bwd_workspace_bytes(ctypes.byref(p), ctypes.byref(bm)))
    if nws == 0:
        _lib.check(lib.mattn_validate(ctypes.byref(p), ctypes.byref(bm)), "mattn_bwd")
    ws, wptr = _workspace(max(nws, 256), q.device)
    _lib.check(lib.mattn_bwd(ctypes.byref(p), ctypes.byref(bm), q.data_ptr(), k.data_ptr(),
                             v.data_ptr(), o.data_ptr(), do.data_ptr(), lse.data_ptr(), _aligned(res),
                             wptr, max(nws, 256), dq.data_ptr(), dk.data_ptr(), dv.data_ptr(),
                             _stream(q.device)),
               "mattn_bwd")
    return dq, dk, dv


class _MaskedAttention(torch.autograd.Function):
    """The reference's custom_vjp (attention.py:180, 244-345).  Residuals are
    (Q, K, V, O, LSE) instead of (Q, K, V): the backward reads the saved
    log-sum-exp rather than re-running the forward scan.

    O is always computed and saved in float32 (the reference's own output
    dtype); a 16-bit ``out_dtype`` is a rounded copy of it.  The backward's
    delta = rowsum(dO * O) then uses the unrounded O: where one key dominates
    a row, dS = P (dP - delta) cancels, and a bfloat16 O would leave its
    rounding (2^-9 of |V|) in dQ and dK."""

    @staticmethod
    def forward(ctx, q, k, v, tm, scale, out_dtype, heads_major=False, precise=False):
        grads = any(ctx.needs_input_grad[:3])
        o, lse, res = mattn_forward(q, k, v, tm, scale, torch.float32, heads_major, for_backward=grads,
                                    precise=precise)
        ctx.save_for_backward(q, k, v, o, lse)
        ctx.tm, ctx.scale, ctx.res, ctx.precise = tm, scale, res, precise
        return o if out_dtype == torch.float32 else o.to(out_dtype)

    @staticmethod
    def backward(ctx, do):
        q, k, v, o, lse = ctx.saved_tensors
        do = _ready(do.to(o.dtype))
        dq, dk, dv = mattn_backward(q, k, v, o, lse, do, ctx.tm, ctx.scale, ctx.res, ctx.precise)
        return dq, dk, dv, None, None, None, None, None


def _kernel_dim(d: int) -> int:
    """Head dimension the kernels run at: 64, 128, 256 or 512 (d zero-padded up to it)."""
    for D in (64, 128, 256, 512):
        if d <= D:
            return D
    raise NotImplementedError(f"head dimension {d} > 512 is not supported by the HIP kernels")


def _pad_dim(x: torch.Tensor, D: int) -> torch.Tensor:
    return x if x.shape[-1] == D else torch.nn.functional.pad(x, (0, D - x.shape[-1]))


PRECISIONS = (None, "default", "highest")


def use_precise(precision: Optional[str], scale: float, d: int) -> bool:
    """Whether a problem runs with MATTN_PRECISE.

    "default": 16-bit inputs run on the MFMA kernels, whose computed operands
    (P, dS, dO) are rounded to float16, 11 significant bits; float32 inputs on
    the float32 SIMT kernels.  "highest": the float32 SIMT kernels for every
    dtype, with the scores formed as compensated dot products (about twice
    float32's precision).  None picks "highest" for kernels sharper than the
    default scale 1/sqrt(d) (threshold_kernel's is 1, attention.py:18-36):
    their logits spread sqrt(d) times wider, rows concentrate on single keys,
    dS = P (dP - delta) cancels below what 11-bit operands resolve, and scores
    of tens of units carry float32's own rounding into the weights."""
    if precision not in PRECISIONS:
        raise ValueError(f"precision must be one of {PRECISIONS}, got {precision!r}")
    if precision is None:
        return abs(scale) > (1.0 + 1e-6) / math.sqrt(d)
    return precision == "highest"


def residue_pack(L: int, P: int) -> int:
    """How many residue classes c one rewritten problem carries: the largest
    power of two dividing P with c L / P <= 128, so that a problem of c L / P
    positions fills (at most) one 128 x 128 tile instead of padding L / P
    rows to 128.  Rows of a problem are positions t (P / c) + r', classes
    r' and r' + P / c, ... interleaved: step t of class r' + (t mod c) P / c."""
    n, c = L // P, 1
    while P % (2 * c) == 0 and 2 * c * n <= bmap.TILE:
        c *= 2
    return c


def residue_problem(L: int, P: int, causal: bool):
    """(view period, keyword arguments of the rewritten call) for the mask
    k % P == q % P (and k <= q) on L positions: the tensors are viewed with
    residue_view(x, P / c), and the c classes a problem interleaves are told
    apart by (t_q - t_k) % c == 0 on its own positions t (with t_k <= t_q for
    causal), c = residue_pack(L, P)."""
    from . import masks

    c = residue_pack(L, P)
    if c == 1:
        return P, dict(is_causal=causal)
    inner = masks.same_residue(c)
    if causal:
        inner = masks.intersect(inner, masks.causal())
    return P // c, dict(mask_fn=inner)


def _residue_rewrite(Q, K, V, is_causal, kernel_fn, mask_fn, block_size, window_size, out_dtype,
                     precision):
    """The strided mask of the reference's benchmark, k % P == q % P (and
    k <= q: check_attn.py:9-32), as independent problems of L / P positions per
    residue class, c classes per problem (residue_pack).

    Position q = s P + r is step s of residue class r, and a query attends only
    keys of its own class, so the [1, L, H, d] tensors viewed as
    [P / c, c L / P, H, d] (batch r', stride H d; position t, stride (P / c) H d:
    views, no copy) carry the same attention under the mask
    (t_q - t_k) % c == 0 (and t_k <= t_q): position t of batch r' is
    t (P / c) + r', and two such positions share a class exactly when
    c divides t_q - t_k.  The tiles of the original problem each hold one
    allowed key per row in 128 (every present tile partial); the rewritten
    problem fills its tile.  Applies to a closed-form mask
    (jaxmodules_amd.masks) that is a residue class, with or without causal,
    and nothing else, no window_size, B = 1 (or 3-D inputs), equal query and
    key lengths divisible by P; None otherwise."""
    from . import masks

    spec = masks.spec_of(mask_fn) if mask_fn is not None else None
    if (spec is None or is_causal or window_size is not None or spec.period is None or spec.period <= 1
            or spec.win_left is not None or spec.win_right is not None or spec.doc_q is not None
            or spec.table is not None):
        return None
    three = Q.dim() == 3
    q4, k4, v4 = (x[None] if three else x for x in (Q, K, V))
    if q4.dim() != 4 or k4.dim() != 4 or v4.dim() != 4:
        return None
    B, N, Hq, d = q4.shape
    L, P = k4.shape[1], spec.period
    if B != 1 or N != L or L % P or v4.shape[1] != L:
        return None
    Pv, inner = residue_problem(L, P, spec.causal)
    if Pv == 1:  # one problem: the original one
        return None
    # the reference's checks (and exception types) on the original call
    bmap.make_plan(tuple(Q.shape), tuple(K.shape), tuple(V.shape), mask_fn=mask_fn,
                   block_size=block_size, window_size=window_size)
    out = _via_map(*(residue_view(x, Pv) for x in (q4, k4, v4)), kernel_fn=kernel_fn, block_size=None,
                   window_size=None, out_dtype=out_dtype, precision=precision, **inner)
    out = residue_unview(out)
    return out[0] if three else out


def residue_view(x: torch.Tensor, P: int) -> torch.Tensor:
    """[1, L, H, d] -> the [P, L / P, H, d] view whose [r, s] is position s P + r."""
    return x[0].reshape(x.shape[1] // P, P, x.shape[2], x.shape[3]).transpose(0, 1)


def residue_unview(y: torch.Tensor) -> torch.Tensor:
    """The inverse of residue_view: [P, n, H, d] -> [1, n P, H, d]."""
    return y.transpose(0, 1).reshape(1, y.shape[0] * y.shape[1], y.shape[2], y.shape[3])


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
    precision: Optional[str] = None,
) -> torch.Tensor:
    """Memory-efficient masked attention (attention.py:347-455).

    K: [B, L, Hkv, d] or [L, Hkv, d]; Q: [B, N, Hq, d] or [N, Hq, d]; V like K.
    is_causal: mask q >= k (exclusive with mask_fn, ValueError otherwise).
    kernel_fn: exp(s * q.k + c): default_kernel (softmax with scale 1/sqrt(d)),
        threshold_kernel(t) (scale 1) or a user kernel of that form, whose s
        is probed (kernel_scale); kernels of any other form raise
        NotImplementedError.
    mask_fn: boolean function of (b, h, q, k) or (h, q, k), elementwise in its
        index arguments (it is evaluated on broadcast numpy index arrays).
    block_size / window_size: as the reference: the window is block-granular,
        clamped at the sequence edges, and may change results (attention.py:374-381).
    out_dtype: dtype of the output.  Default float32, which is what the
        reference returns (its running accumulators are float32,
        attention.py:173); pass Q.dtype for a 16-bit output.
    precision: None, "default" or "highest" (use_precise): 16-bit inputs run
        on float16-operand MFMA kernels by default and in float32 arithmetic
        (compensated scores) with "highest", which None selects for kernels
        sharper than default_kernel (threshold_kernel).  Not a reference
        argument.

    Returns [B, N, Hq, d] (or [N, Hq, d]); differentiable w.r.t. Q, K, V.
    Rows with no allowed key are zero (attention.py:91-100).

    A residue-class mask (masks.same_residue, with or without masks.causal:
    the reference benchmark's, check_attn.py:9-32) runs as L / P-long problems
    over strided views (_residue_rewrite).
    """
    rw = _residue_rewrite(Q, K, V, is_causal, kernel_fn, mask_fn, block_size, window_size, out_dtype, precision)
    if rw is not None:
        return rw
    return _via_map(Q, K, V, is_causal=is_causal, kernel_fn=kernel_fn, mask_fn=mask_fn, block_size=block_size,
                    window_size=window_size, out_dtype=out_dtype, precision=precision)


def _via_map(Q, K, V, *, is_causal=False, kernel_fn=default_kernel, mask_fn=None, block_size=None,
             window_size=None, out_dtype=None, precision=None):
    """masked_attention_via_map without the residue-class rewrite."""
    plan, tm = trace_call(tuple(Q.shape), tuple(K.shape), tuple(V.shape), is_causal=is_causal,
                          mask_fn=mask_fn, block_size=block_size, window_size=window_size,
                          device=Q.device if Q.is_cuda else None)
    scale = kernel_scale(kernel_fn, plan.d)
    if not (Q.is_cuda and K.is_cuda and V.is_cuda):
        raise RuntimeError("masked_attention_via_map runs on the GPU only (no CPU code path)")
    dt = torch.promote_types(torch.promote_types(Q.dtype, K.dtype), V.dtype)
    if dt not in _DT:
        raise TypeError(f"unsupported dtype {dt}")
    if plan.squeeze_batch:
        Q, K, V = Q[None], K[None], V[None]
    D = _kernel_dim(plan.d)
    Q = Q.to(dt)
    # softmax(s q.k) == softmax(|s| (-q).k); s == 0 gives uniform weights: q = 0, scale 1
    if scale < 0:
        Q, scale = -Q, -scale
    elif scale == 0:
        Q, scale = Q * 0, 1.0
    precise = use_precise(precision, scale, plan.d)
    q, k, v = (_ready(_pad_dim(x.to(dt), D)) for x in (Q, K, V))
    od = _out_dtype(dt, out_dtype)
    out = _MaskedAttention.apply(q, k, v, tm, scale, od, False, precise)
    if D != plan.d:
        out = out[..., :plan.d]
    return out[0] if plan.squeeze_batch else out


def _out_dtype(dt, out_dtype):
    od = torch.float32 if out_dtype is None else out_dtype
    if dt == torch.float32 and od != torch.float32:
        raise TypeError("float32 inputs produce a float32 output")
    if od not in (torch.float32, dt):
        raise TypeError(f"out_dtype must be float32 or {dt}")
    return od


# ---------------------------------------------------------------------------
# flex_attention (attention.py:456-692)
# ---------------------------------------------------------------------------

_BM_CACHE: "OrderedDict[tuple, bmap.TileMap]" = OrderedDict()


def _block_mask_tiles(block_mask, B, Hq, Hkv, L, S, element_head="kv") -> bmap.TileMap:
    """Tile map of a BlockMask (or of the full mask when None), cached per mask
    object and head layout."""
    from .block_mask import BlockMask

    # the launch orders of a tile map are laid out for (B, Hq, Hkv): part of the key
    key = ("full", L, S, B, Hq, Hkv) if block_mask is None else (block_mask, B, Hq, Hkv, element_head)
    tm = _BM_CACHE.get(key)
    if tm is None:
        if block_mask is None:
            tm = BlockMask.full_mask(1, 1, L, S, (L, S)).tile_map(B, Hq, Hkv)
        else:
            tm = block_mask.tile_map(B, Hq, Hkv, element_head)
        _BM_CACHE[key] = tm
        if len(_BM_CACHE) > _CACHE_SIZE:
            _BM_CACHE.popitem(last=False)
    else:
        _BM_CACHE.move_to_end(key)
    return tm


def flex_attention(query: torch.Tensor, key: torch.Tensor, value: torch.Tensor,
                   score_mod: Optional[Callable] = None, block_mask=None, scale=None,
                   enable_gqa: bool = False, return_lse: bool = False,
                   out_dtype: Optional[torch.dtype] = None, *, precision: Optional[str] = None,
                   _element_head: str = "kv") -> torch.Tensor:
    """Block-sparse softmax attention over a ``BlockMask`` (attention.py:456-692).

    query [B, Hq, L, E], key [B, Hkv, S, E], value [B, Hkv, S, E]; returns
    [B, Hq, L, E] (float32 by default, like the reference's float32 running
    accumulators; ``out_dtype`` = the input dtype for a 16-bit output),
    differentiable w.r.t. query, key and value.  Query head hq reads KV head
    hq // (Hq / Hkv).  The attention pattern is the block mask's: full tiles
    whole, partial tiles where ``mask_mod`` holds (``BlockMask.tile_map`` gives
    the element rule); no block mask means every key.  Rows with no allowed key
    are zero (attention.py:598-617).

    Same checks and exception types as the reference (AssertionError for shape
    mismatches, NotImplementedError for ``return_lse``).  ``score_mod`` has no
    kernel here and raises NotImplementedError, as does a value head dimension
    different from the query's.  ``precision`` as for masked_attention_via_map
    (None selects float32 arithmetic for a ``scale`` above 1/sqrt(E)).
    """
    if return_lse:
        raise NotImplementedError("return_lse is not supported yet")
    B, Hq, L, E = query.shape
    Bk, Hkv, S, Ek = key.shape
    Bv, Hv, Sv, Ev = value.shape
    assert E == Ek, "query and key must have the same embedding dimension"
    assert B == Bk, "query and key must have the same batch dimension"
    assert Sv == S, "value and key must have the same sequence length"
    assert Bv == B, "value and query must have the same batch dimension"
    assert Hv == Hkv, "value and key must have the same head count"
    if block_mask is not None:
        Qb, KVb = block_mask.Q_BLOCK_SIZE, block_mask.KV_BLOCK_SIZE
        assert L == block_mask.Q_LEN, "query length must match block mask"
        assert S == block_mask.KV_LEN, "key length must match block mask"
        assert L % Qb == 0, "query length must be divisible by Q_BLOCK_SIZE"
        assert S % KVb == 0, "key length must be divisible by KV_BLOCK_SIZE"
    if not enable_gqa:
        assert Hq == Hkv, "query and key must have the same head count, unless enable_gqa is True"
    assert Hq % Hkv == 0, "kv head count must divide query head count"
    if score_mod is not None:
        raise NotImplementedError("score_mod is not supported by the HIP kernels")
    if Ev != E:
        raise NotImplementedError("value head dimension must equal the query/key head dimension")
    if not (query.is_cuda and key.is_cuda and value.is_cuda):
        raise RuntimeError("flex_attention runs on the GPU only (no CPU code path)")
    dt = torch.promote_types(torch.promote_types(query.dtype, key.dtype), value.dtype)
    if dt not in _DT:
        raise TypeError(f"unsupported dtype {dt}")
    s = 1.0 / math.sqrt(E) if scale is None else float(scale)
    if not math.isfinite(s):
        raise ValueError(f"scale must be finite, got {s}")
    precise = use_precise(precision, s, E)
    tm = _block_mask_tiles(block_mask, B, Hq, Hkv, L, S, _element_head)
    D = _kernel_dim(E)
    q = query.to(dt)
    # softmax(s q.k) == softmax(|s| (-q).k); s == 0 gives uniform weights: q = 0, scale 1
    if s < 0:
        q, s = -q, -s
    elif s == 0:
        q, s = q * 0, 1.0
    # [B, H, L, E] tensors are strided [B, L, H, E] views for the kernels
    q, k, v = (_ready(_pad_dim(x, D).transpose(1, 2)) for x in (q, key.to(dt), value.to(dt)))
    out = _MaskedAttention.apply(q, k, v, tm, s, _out_dtype(dt, out_dtype), True, precise)
    out = out.transpose(1, 2)
    return out[..., :E] if D != E else out


def flex_attention_slow(query, key, value, score_mod=None, block_mask=None, scale=None,
                        enable_gqa=False, return_lse=False, out_dtype=None, precision=None):
    """The reference's materialised-mask variant (attention.py:695-820) on the
    same kernels.  As there: Hq != Hkv is accepted without ``enable_gqa``,
    ``return_lse`` is ignored, and partial-tile elements are evaluated with the
    query head (``materialize_mask``).  A row with no allowed key is zero here;
    the reference's softmax over an all -inf row gives NaN."""
    return flex_attention(query, key, value, score_mod=score_mod, block_mask=block_mask,
                          scale=scale, enable_gqa=True, out_dtype=out_dtype, precision=precision,
                          _element_head="query")
