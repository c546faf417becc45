"""ctypes binding of ``libmattn.so`` (declarations in ``include/mattn.h``).

The library is loaded from the package directory (built in-tree by
``jaxmodules_amd.build``).  There is no fallback: if the library is missing the
import of ``load()`` raises, so no attention call can silently run elsewhere.
"""
from __future__ import annotations

import ctypes
import os
import threading

# MATTN_LIBRARY selects another build of the same library (e.g. to compare
# compiler settings); the default is the in-tree build.
LIB_PATH = os.environ.get("MATTN_LIBRARY") or os.path.join(
    os.path.dirname(os.path.abspath(__file__)), "libmattn.so")

MATTN_BF16, MATTN_F16, MATTN_F32 = 0, 1, 2
MATTN_FWD_FOR_BWD = 1
MATTN_BWD_DS = 2
MATTN_PRECISE = 4
TILE_Q = TILE_K = 128
ABI_VERSION = 8

STATUS = {
    0: "MATTN_OK",
    -1: "MATTN_ERR_NULL",
    -2: "MATTN_ERR_SHAPE",
    -3: "MATTN_ERR_HEAD_DIM",
    -4: "MATTN_ERR_DTYPE",
    -5: "MATTN_ERR_STRIDE",
    -6: "MATTN_ERR_BLOCKMAP",
    -7: "MATTN_ERR_LAUNCH",
    -8: "MATTN_ERR_TOO_LARGE",
    -9: "MATTN_ERR_SCRATCH",
    -10: "MATTN_ERR_DEVICE",
    -11: "MATTN_ERR_WORKSPACE",
    -12: "MATTN_ERR_RESIDUAL",
}

# every symbol include/mattn.h declares
EXPORTS = ("mattn_validate", "mattn_workspace_bytes", "mattn_bwd_workspace_bytes", "mattn_fwd_workspace_bytes",
           "mattn_fwd", "mattn_bwd",
           "mattn_bwd_stage", "mattn_strerror", "mattn_abi_version", "mattn_maskspec_validate",
           "mattn_tilemap_classify", "mattn_tilemap_bits", "mattn_bwd_noalloc")
SCRATCH_BYTES = 512 << 20  # MATTN_SCRATCH_BYTES
BWD_PRE, BWD_DKDV, BWD_DQ = 0, 1, 2

_I64x3 = ctypes.c_int64 * 3


class MattnProblem(ctypes.Structure):
    _fields_ = [
        ("B", ctypes.c_int32), ("Lq", ctypes.c_int32), ("Lk", ctypes.c_int32),
        ("Hq", ctypes.c_int32), ("Hkv", ctypes.c_int32), ("D", ctypes.c_int32),
        ("dtype", ctypes.c_int32), ("o_dtype", ctypes.c_int32),
        ("scale", ctypes.c_float), ("flags", ctypes.c_int32),
        ("q_stride", _I64x3), ("k_stride", _I64x3), ("v_stride", _I64x3), ("o_stride", _I64x3),
        ("do_stride", _I64x3), ("dq_stride", _I64x3), ("dk_stride", _I64x3), ("dv_stride", _I64x3),
    ]


class MattnBlockmap(ctypes.Structure):
    _fields_ = [
        ("map_b", ctypes.c_int32), ("map_h", ctypes.c_int32),
        ("nqt", ctypes.c_int32), ("nkt", ctypes.c_int32),
        ("n_masks", ctypes.c_int32), ("nnz", ctypes.c_int32),
        ("row_ptr", ctypes.c_void_p), ("row_ent", ctypes.c_void_p),
        ("col_ptr", ctypes.c_void_p), ("col_ent", ctypes.c_void_p),
        ("row_bits", ctypes.c_void_p), ("col_bits", ctypes.c_void_p),
        ("q_order", ctypes.c_void_p), ("kv_order", ctypes.c_void_p),
        ("n_q_order", ctypes.c_int32), ("n_kv_order", ctypes.c_int32),
        ("col_row", ctypes.c_void_p), ("kv_desc", ctypes.c_void_p),
    ]


class MattnMaskspec(ctypes.Structure):
    _fields_ = [
        ("causal", ctypes.c_int32), ("win_left", ctypes.c_int32), ("win_right", ctypes.c_int32),
        ("doc_b", ctypes.c_int32), ("doc_q", ctypes.c_void_p), ("doc_k", ctypes.c_void_p),
        ("tab_b", ctypes.c_int32), ("tab_h", ctypes.c_int32), ("tiles", ctypes.c_void_p),
        ("blk_size", ctypes.c_int32), ("blk_left", ctypes.c_int32), ("blk_right", ctypes.c_int32),
        ("blk_nk", ctypes.c_int32), ("res_period", ctypes.c_int32),
    ]


class MattnError(RuntimeError):
    def __init__(self, code: int, what: str = ""):
        self.code = code
        text = load().mattn_strerror(code).decode()
        super().__init__(f"{what}: {STATUS.get(code, code)} ({text})" if what else text)


_lib = None
_lock = threading.Lock()


def load():
    """Loads the library once; raises ImportError when it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not os.path.exists(LIB_PATH):
            raise ImportError(
                f"{LIB_PATH} is missing: build it with `python -m jaxmodules_amd.build` "
                "(the masked attention has no non-HIP code path)")
        lib = ctypes.CDLL(LIB_PATH)
        P = ctypes.POINTER(MattnProblem)
        M = ctypes.POINTER(MattnBlockmap)
        vp = ctypes.c_void_p
        lib.mattn_validate.argtypes = [P, M]
        lib.mattn_validate.restype = ctypes.c_int
        lib.mattn_workspace_bytes.argtypes = [P]
        lib.mattn_workspace_bytes.restype = ctypes.c_size_t
        lib.mattn_bwd_workspace_bytes.argtypes = [P, M]
        lib.mattn_bwd_workspace_bytes.restype = ctypes.c_size_t
        lib.mattn_fwd_workspace_bytes.argtypes = [P]
        lib.mattn_fwd_workspace_bytes.restype = ctypes.c_size_t
        lib.mattn_fwd.argtypes = [P, M, vp, vp, vp, vp, vp, vp, vp]
        lib.mattn_fwd.restype = ctypes.c_int
        sz = ctypes.c_size_t
        lib.mattn_bwd.argtypes = [P, M, vp, vp, vp, vp, vp, vp, vp, vp, sz, vp, vp, vp, vp]
        lib.mattn_bwd.restype = ctypes.c_int
        lib.mattn_bwd_stage.argtypes = [P, M, ctypes.c_int, vp, vp, vp, vp, vp, vp, vp, vp, sz, vp, vp, vp, vp]
        lib.mattn_bwd_noalloc.argtypes = [P, M, vp, vp, vp, vp, vp, vp, vp, vp, vp, vp, vp]
        lib.mattn_bwd_noalloc.restype = ctypes.c_int
        lib.mattn_bwd_stage.restype = ctypes.c_int
        lib.mattn_strerror.argtypes = [ctypes.c_int]
        lib.mattn_strerror.restype = ctypes.c_char_p
        S = ctypes.POINTER(MattnMaskspec)
        i32 = ctypes.c_int32
        lib.mattn_maskspec_validate.argtypes = [S, i32, i32, i32, i32]
        lib.mattn_maskspec_validate.restype = ctypes.c_int
        lib.mattn_tilemap_classify.argtypes = [S, i32, i32, i32, i32, vp, vp, vp, vp]
        lib.mattn_tilemap_classify.restype = ctypes.c_int
        lib.mattn_tilemap_bits.argtypes = [S, i32, i32, i32, i32, vp, i32, i32, i32, vp, vp, vp, vp]
        lib.mattn_tilemap_bits.restype = ctypes.c_int
        lib.mattn_abi_version.argtypes = []
        lib.mattn_abi_version.restype = ctypes.c_int
        if lib.mattn_abi_version() != ABI_VERSION:
            raise ImportError(f"{LIB_PATH}: ABI version {lib.mattn_abi_version()} != {ABI_VERSION}")
        _lib = lib
    return _lib


def check(code: int, what: str = ""):
    if code != 0:
        raise MattnError(code, what)
