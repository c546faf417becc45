"""The C ABI without a GPU: the library loads, exports every symbol
include/mattn.h declares, its structs match the header byte for byte, and the
host-only validation returns the documented codes."""
import ctypes
import os
import re
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "mattn.h")

from jaxmodules_amd import _lib  # noqa: E402


@pytest.fixture(scope="module")
def lib():
    if not os.path.exists(_lib.LIB_PATH):
        pytest.skip("libmattn.so not built (run __graft_entry__.build())")
    return _lib.load()


def declared_functions():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"^\s*(?:int|size_t|const char\*)\s+(mattn_\w+)\s*\(", text, re.M)))


def test_header_declares_exports():
    assert declared_functions() == sorted(_lib.EXPORTS)


def test_library_exports_every_symbol(lib):
    out = subprocess.run(["nm", "-D", "--defined-only", _lib.LIB_PATH], capture_output=True,
                         text=True, check=True).stdout
    syms = {l.split()[-1] for l in out.splitlines() if " T " in l}
    for name in declared_functions():
        assert name in syms, name
        assert hasattr(lib, name)


def test_abi_version(lib):
    assert lib.mattn_abi_version() == _lib.ABI_VERSION


def test_struct_layout_matches_header(tmp_path):
    """Compile a probe against the header and compare sizeof/offsetof with ctypes."""
    fields = {"mattn_problem": _lib.MattnProblem, "mattn_blockmap": _lib.MattnBlockmap,
              "mattn_maskspec": _lib.MattnMaskspec}
    lines = ['#include <stdio.h>', '#include <stddef.h>', '#include "mattn.h"', "int main(void){"]
    for cname, cls in fields.items():
        lines.append(f'printf("{cname} sizeof %zu\\n", sizeof({cname}));')
        for f, _ in cls._fields_:
            lines.append(f'printf("{cname} {f} %zu\\n", offsetof({cname}, {f}));')
    lines.append("return 0;}")
    src = tmp_path / "probe.c"
    src.write_text("\n".join(lines))
    exe = tmp_path / "probe"
    subprocess.run(["gcc", "-std=c11", "-I", os.path.dirname(HEADER), str(src), "-o", str(exe)],
                   check=True)
    got = {}
    for l in subprocess.run([str(exe)], capture_output=True, text=True, check=True).stdout.splitlines():
        c, f, v = l.split()
        got[(c, f)] = int(v)
    for cname, cls in fields.items():
        assert got[(cname, "sizeof")] == ctypes.sizeof(cls), cname
        for f, _ in cls._fields_:
            assert got[(cname, f)] == getattr(cls, f).offset, (cname, f)


def _problem(**kw):
    p = _lib.MattnProblem(B=2, Lq=300, Lk=300, Hq=8, Hkv=2, D=128, dtype=_lib.MATTN_BF16,
                          o_dtype=_lib.MATTN_F32, scale=0.088)
    for name in ("q", "k", "v", "dq", "dk", "dv"):
        setattr(p, f"{name}_stride", (ctypes.c_int64 * 3)(300 * 8 * 128, 8 * 128, 128))
    for name in ("o", "do"):
        setattr(p, f"{name}_stride", (ctypes.c_int64 * 3)(300 * 8 * 128, 8 * 128, 128))
    for k, v in kw.items():
        setattr(p, k, v)
    return p


def _validate(lib, p, bm=None):
    return lib.mattn_validate(ctypes.byref(p), ctypes.byref(bm) if bm is not None else None)


def test_validate_codes(lib):
    assert _validate(lib, _problem()) == 0
    assert _validate(lib, _problem(Hkv=3)) == -2          # Hq % Hkv
    assert _validate(lib, _problem(B=0)) == -2
    assert _validate(lib, _problem(D=96)) == -3
    assert _validate(lib, _problem(D=256)) == 0
    assert _validate(lib, _problem(D=512)) == 0
    assert _validate(lib, _problem(D=1024)) == -3
    assert _validate(lib, _problem(dtype=7)) == -4
    assert _validate(lib, _problem(dtype=_lib.MATTN_F32, o_dtype=_lib.MATTN_BF16)) == -4
    assert _validate(lib, _problem(o_dtype=_lib.MATTN_F16)) == -4   # bf16 in, fp16 out
    p = _problem()
    p.q_stride = (ctypes.c_int64 * 3)(300 * 8 * 128, 8 * 128 + 3, 128)
    assert _validate(lib, p) == -5
    assert lib.mattn_validate(None, None) == -1
    for code in (0, -1, -2, -3, -4, -5, -6, -7, -8, -9, -10, 123):
        assert isinstance(lib.mattn_strerror(code), bytes)


def test_validate_blockmap(lib):
    p = _problem()
    bm = _lib.MattnBlockmap(map_b=1, map_h=1, nqt=3, nkt=3, n_masks=0, nnz=0, row_ptr=8, col_ptr=8,
                            q_order=8, kv_order=8, n_q_order=2 * 8 * 3, n_kv_order=2 * 2 * 3)
    assert _validate(lib, p, bm) == 0
    bm.nqt = 2
    assert _validate(lib, p, bm) == -6
    bm.nqt = 3
    bm.map_h = 4
    assert _validate(lib, p, bm) == -6
    bm.map_h = 8
    assert _validate(lib, p, bm) == 0
    bm.n_q_order = 10
    assert _validate(lib, p, bm) == -6
    bm.n_q_order = 48
    bm.nnz = 5
    assert _validate(lib, p, bm) == -1                     # entries missing
    bm.row_ent = bm.col_ent = 8
    bm.n_masks = 1
    assert _validate(lib, p, bm) == -1                     # bit arrays missing


def test_workspace_bytes(lib):
    """The documented layouts.  Backward workspace: delta, then (16-bit
    inputs) the shifted lse, float16 dO' padded to whole 128-row tiles per
    head, float16 K' per kv-head tile, and per tile the dO' scale, dS bounds
    (2 floats), dS scale and K' scale; then for the split tiles the
    rounded-off part of dO' (float16, like dO') and the unrounded dK and dV
    of a key tile (float32, 2 x 128 x D per key tile).  Forward residual:
    float16 V' and Q', then V' scales and maxima, Q' scales, each query
    tile's largest attention weight and its 128-bit mask of split rows, and a
    flag per key tile (a split row has an allowed key there)."""
    align = lambda x: (x + 255) // 256 * 256
    B, L, Hq, Hkv, D = 2, 300, 8, 2, 128
    nqt = -(-L // 128)
    qtiles, ktiles = B * Hq * nqt, B * Hkv * nqt
    want = (2 * align(B * Hq * L * 4) + align(qtiles * 128 * D * 2) + align(ktiles * 128 * D * 2)
            + align(qtiles * 4) + align(qtiles * 8) + align(qtiles * 4) + align(ktiles * 4)
            + align(qtiles * 128 * D * 2) + align(ktiles * 2 * 128 * D * 4))
    p = _problem()
    assert lib.mattn_workspace_bytes(ctypes.byref(p)) == want
    p16 = _problem(dtype=_lib.MATTN_F16, o_dtype=_lib.MATTN_F16)
    assert lib.mattn_workspace_bytes(ctypes.byref(p16)) == want
    p32 = _problem(dtype=_lib.MATTN_F32, o_dtype=_lib.MATTN_F32)
    assert lib.mattn_workspace_bytes(ctypes.byref(p32)) == align(B * Hq * L * 4)
    res = (align(ktiles * 128 * D * 2) + align(qtiles * 128 * D * 2) + 2 * align(ktiles * 4)
           + 2 * align(qtiles * 4) + align(qtiles * 16) + align(ktiles * 4))
    assert lib.mattn_fwd_workspace_bytes(ctypes.byref(p)) == res
    assert lib.mattn_fwd_workspace_bytes(ctypes.byref(p32)) == 0
    assert lib.mattn_workspace_bytes(ctypes.byref(_problem(D=80))) == 0
    assert lib.mattn_fwd_workspace_bytes(ctypes.byref(_problem(D=80))) == 0
    # D = 256 runs on the float32 SIMT kernels for every dtype: delta only, no residual
    for dt in (_lib.MATTN_BF16, _lib.MATTN_F16, _lib.MATTN_F32):
        p256 = _problem(D=256, dtype=dt, o_dtype=dt)
        assert lib.mattn_workspace_bytes(ctypes.byref(p256)) == align(B * Hq * L * 4)
        assert lib.mattn_fwd_workspace_bytes(ctypes.byref(p256)) == 0


def test_flags_validated(lib):
    assert _validate(lib, _problem(flags=_lib.MATTN_FWD_FOR_BWD)) == 0
    assert _validate(lib, _problem(flags=_lib.MATTN_BWD_DS)) == 0
    assert _validate(lib, _problem(flags=_lib.MATTN_FWD_FOR_BWD | _lib.MATTN_BWD_DS)) == 0
    assert _validate(lib, _problem(flags=_lib.MATTN_PRECISE)) == 0
    assert _validate(lib, _problem(flags=8)) == -2


def test_bwd_workspace_bytes_with_stored_ds(lib):
    """mattn_bwd_workspace_bytes: the plain workspace, plus with MATTN_BWD_DS
    32 KiB per present tile of every (batch, head) the map covers -- the map's
    nnz tiles once per (b, h) it is broadcast over."""
    p = _problem()                                   # B=2, Hq=8, L=300: nqt = nkt = 3
    base = lib.mattn_workspace_bytes(ctypes.byref(p))
    bm = _lib.MattnBlockmap(map_b=1, map_h=1, nqt=3, nkt=3, n_masks=0, nnz=6, row_ptr=8, col_ptr=8,
                            row_ent=8, col_ent=8, col_row=8, q_order=8, kv_order=8,
                            n_q_order=2 * 8 * 3, n_kv_order=2 * 2 * 3)
    assert lib.mattn_bwd_workspace_bytes(ctypes.byref(p), ctypes.byref(bm)) == base
    p.flags = _lib.MATTN_BWD_DS
    assert lib.mattn_bwd_workspace_bytes(ctypes.byref(p), ctypes.byref(bm)) == base + 6 * 2 * 8 * 32768
    bm.map_h = 8                                      # per-head map: its nnz covers every head
    assert lib.mattn_bwd_workspace_bytes(ctypes.byref(p), ctypes.byref(bm)) == base + 6 * 2 * 32768
    bm.map_b = 2
    assert lib.mattn_bwd_workspace_bytes(ctypes.byref(p), ctypes.byref(bm)) == base + 6 * 32768
    # the float32 (SIMT) path ignores the flag
    p32 = _problem(dtype=_lib.MATTN_F32, o_dtype=_lib.MATTN_F32, flags=_lib.MATTN_BWD_DS)
    assert lib.mattn_bwd_workspace_bytes(ctypes.byref(p32), ctypes.byref(bm)) == \
        lib.mattn_workspace_bytes(ctypes.byref(p32))
    # an invalid map or problem gives 0
    assert lib.mattn_bwd_workspace_bytes(ctypes.byref(p), None) == 0
    bm.nqt = 2
    assert lib.mattn_bwd_workspace_bytes(ctypes.byref(p), ctypes.byref(bm)) == 0
    # the stored dS needs the column entries' row indices
    bm.nqt = 3
    bm.col_row = None
    p.flags |= _lib.MATTN_FWD_FOR_BWD
    need = lib.mattn_bwd_workspace_bytes(ctypes.byref(p), ctypes.byref(bm))
    assert lib.mattn_bwd_stage(ctypes.byref(p), ctypes.byref(bm), 1, 8, 8, 8, 8, 8, 8, 256, 256, need,
                               8, 8, 8, None) == -1


def test_dkdv_stage_needs_the_launch_descriptors(lib):
    """The MFMA dK/dV stage reads kv_desc (one row per launch slot); without it
    the call returns MATTN_ERR_NULL before any launch.  The float32 (SIMT)
    path does not read it."""
    p = _problem()
    bm = _lib.MattnBlockmap(map_b=1, map_h=1, nqt=3, nkt=3, n_masks=0, nnz=0, row_ptr=8, col_ptr=8,
                            q_order=8, kv_order=8, n_q_order=2 * 8 * 3, n_kv_order=2 * 2 * 3, kv_desc=None)
    p.flags = _lib.MATTN_FWD_FOR_BWD
    ptrs = [8, 8, 8, 8, 8, 8, 256, 256, 1 << 30, 8, 8, 8]
    assert lib.mattn_bwd_stage(ctypes.byref(p), ctypes.byref(bm), _lib.BWD_DKDV, *ptrs, None) == -1


def test_heads_major_long_sequences_validate(lib):
    """Heads-major views (flex_attention's layout) with Hq * Lq * D >= 2^31: the
    float16 dO' and Q' copies the dK/dV kernel reads are head-major, one buffer
    resource per head, so only one head's copy must fit 32-bit byte offsets."""
    Hq, L, D = 128, 262144, 128
    p = _problem(B=1, Lq=L, Lk=L, Hq=Hq, Hkv=Hq)
    hm = (ctypes.c_int64 * 3)(Hq * L * D, D, L * D)          # [B, H, L, D] memory, BLHD view
    for name in ("q", "k", "v", "dq", "dk", "dv", "o", "do"):
        setattr(p, f"{name}_stride", hm)
    assert Hq * L * D * 2 >= 2 ** 31
    assert _validate(lib, p) == 0
    # one head's float16 copy past 2^31 bytes is refused
    L2 = 2 ** 23
    p2 = _problem(B=1, Lq=L2, Lk=128, Hq=1, Hkv=1)
    for name in ("q", "dq", "o", "do"):
        setattr(p2, f"{name}_stride", (ctypes.c_int64 * 3)(L2 * D, D, D))
    for name in ("k", "v", "dk", "dv"):
        setattr(p2, f"{name}_stride", (ctypes.c_int64 * 3)(128 * D, D, D))
    assert _validate(lib, p2) == -8


def test_entry_points_reject_before_launch(lib):
    """Error paths return codes without touching the GPU (no device here)."""
    p = _problem(D=96)
    rc = lib.mattn_fwd(ctypes.byref(p), None, None, None, None, None, None, None, None)
    assert rc == -3
    p = _problem()
    rc = lib.mattn_fwd(ctypes.byref(p), None, None, None, None, None, None, None, None)
    assert rc == -1
    rc = lib.mattn_bwd_stage(ctypes.byref(p), None, 5, *([None] * 8), 0, *([None] * 4))
    assert rc == -1


def test_backward_checks_workspace_size_and_residual_flag(lib):
    """ABI 8: the backward rejects a workspace smaller than
    mattn_bwd_workspace_bytes (MATTN_ERR_WORKSPACE) and, on the MFMA path, a
    problem without MATTN_FWD_FOR_BWD, whose residual holds no float16 Q copy
    (MATTN_ERR_RESIDUAL), both before any launch.  MATTN_PRECISE problems run
    on the SIMT kernels: no residual, a one-float-per-row workspace."""
    p = _problem(flags=_lib.MATTN_FWD_FOR_BWD | _lib.MATTN_BWD_DS)
    bm = _lib.MattnBlockmap(map_b=1, map_h=1, nqt=3, nkt=3, n_masks=0, nnz=4, row_ptr=8, col_ptr=8,
                            row_ent=8, col_ent=8, q_order=8, kv_order=8, n_q_order=2 * 8 * 3,
                            n_kv_order=2 * 2 * 3, col_row=8, kv_desc=8)
    need = lib.mattn_bwd_workspace_bytes(ctypes.byref(p), ctypes.byref(bm))
    ptrs = [8, 8, 8, 8, 8, 8, 256, 256]
    assert lib.mattn_bwd_stage(ctypes.byref(p), ctypes.byref(bm), 0, *ptrs, need - 1, 8, 8, 8, None) == -11
    assert lib.mattn_bwd(ctypes.byref(p), ctypes.byref(bm), *ptrs, need - 1, 8, 8, 8, None) == -11
    p.flags = _lib.MATTN_BWD_DS
    need = lib.mattn_bwd_workspace_bytes(ctypes.byref(p), ctypes.byref(bm))
    assert lib.mattn_bwd_stage(ctypes.byref(p), ctypes.byref(bm), 0, *ptrs, need, 8, 8, 8, None) == -12
    # float32 arithmetic for 16-bit inputs: SIMT path, no residual, no stored dS
    p.flags = _lib.MATTN_PRECISE | _lib.MATTN_BWD_DS
    assert lib.mattn_validate(ctypes.byref(p), ctypes.byref(bm)) == 0
    rows = p.B * p.Hq * p.Lq           # the residual: what each row's lse and O round off
    a256 = lambda x: (x + 255) // 256 * 256  # noqa: E731
    assert lib.mattn_fwd_workspace_bytes(ctypes.byref(p)) == a256(rows * 4) + a256(rows * p.D * 4)
    p32 = _problem(dtype=_lib.MATTN_F32, o_dtype=_lib.MATTN_F32)
    assert lib.mattn_bwd_workspace_bytes(ctypes.byref(p), ctypes.byref(bm)) == \
        lib.mattn_workspace_bytes(ctypes.byref(p32))
    p.flags = 8  # an undefined flag bit
    assert lib.mattn_validate(ctypes.byref(p), None) == -2


def test_library_missing_raises(monkeypatch, tmp_path):
    monkeypatch.setattr(_lib, "LIB_PATH", str(tmp_path / "nope.so"))
    monkeypatch.setattr(_lib, "_lib", None)
    with pytest.raises(ImportError):
        _lib.load()


def test_noalloc_rejects_before_any_device_call(lib):
    """mattn_bwd_noalloc checks the problem and its workspace size against the
    static scratch on the host, before it touches a device."""
    n, h = 32768, 32                     # dO', its rounded-off part and K' copies: 3 x 256 MiB
    p = _problem(B=1, Lq=n, Lk=n, Hq=h, Hkv=h)
    for name in ("q", "k", "v", "dq", "dk", "dv", "o", "do"):
        setattr(p, f"{name}_stride", (ctypes.c_int64 * 3)(n * h * 128, h * 128, 128))
    assert lib.mattn_workspace_bytes(ctypes.byref(p)) > _lib.SCRATCH_BYTES
    args = [None] * 11
    assert lib.mattn_bwd_noalloc(ctypes.byref(p), None, *args) == -9
    assert lib.mattn_bwd_noalloc(ctypes.byref(_problem(D=96)), None, *args) == -3
    small = _problem()
    assert lib.mattn_workspace_bytes(ctypes.byref(small)) <= _lib.SCRATCH_BYTES


def _causal_map(B, L, H):
    """A mattn_blockmap of a causal map broadcast over batch and heads (host
    sizes only; the pointers are never dereferenced)."""
    nt = -(-L // 128)
    return _lib.MattnBlockmap(map_b=1, map_h=1, nqt=nt, nkt=nt, n_masks=1, nnz=nt * (nt + 1) // 2,
                              row_ptr=8, col_ptr=8, row_ent=8, col_ent=8, row_bits=8, col_bits=8,
                              q_order=8, kv_order=8, n_q_order=B * H * nt, n_kv_order=B * H * nt,
                              col_row=8, kv_desc=8)


def test_stored_ds_default_stays_within_its_cap(lib):
    """The default backward keeps dS only while its extra workspace is at most
    attention.DS_MAX_BYTES (4 GiB): B=1 L=8192 H=32 causal (2.2 GB) keeps it,
    L=16384 (8.7 GB, O(L^2)) recomputes dS instead, with the O(L) workspace."""
    from jaxmodules_amd import attention as A

    assert A.STORE_DS is None and A.DS_MAX_BYTES == 4 << 30
    for L, keeps in ((8192, True), (16384, False)):
        p = _problem(B=1, Lq=L, Lk=L, Hq=32, Hkv=32, flags=_lib.MATTN_FWD_FOR_BWD)
        for name in ("q", "k", "v", "dq", "dk", "dv"):
            setattr(p, f"{name}_stride", (ctypes.c_int64 * 3)(L * 32 * 128, 32 * 128, 128))
        for name in ("o", "do"):
            setattr(p, f"{name}_stride", (ctypes.c_int64 * 3)(L * 32 * 128, 32 * 128, 128))
        bm = _causal_map(1, L, 32)
        flags = A.bwd_flags(p, bm)
        assert bool(flags & _lib.MATTN_BWD_DS) == keeps, L
        p.flags = flags
        extra = lib.mattn_bwd_workspace_bytes(ctypes.byref(p), ctypes.byref(bm)) - \
            lib.mattn_workspace_bytes(ctypes.byref(p))
        assert extra <= A.DS_MAX_BYTES
        if not keeps:
            # the recomputing backward's workspace: O(L) per head -- per query row
            # delta and the shifted lse (8 bytes) and the float16 dO' and its
            # rounded-off part (4 D bytes), per key row the float16 K' (2 D bytes)
            # and the split columns' float32 dK and dV (8 D bytes), plus per-tile
            # scales and flags
            rows = L * 32
            assert lib.mattn_workspace_bytes(ctypes.byref(p)) < rows * (8 + 4 * 128) + rows * 10 * 128 + (8 << 20)
