"""Static check of compiled kernel assembly (gfx950): no instruction reads or
overwrites the destination VGPRs of an LDS read before an ``s_waitcnt lgkmcnt``
has covered that read.

The forward, dK/dV and dQ kernels issue their MFMA operand reads as
inline-asm ``ds_read`` instructions with hand-counted waits (the compiler does not track them), so
the waits are checked on the code the compiler actually emitted.  LDS reads
complete in order, so ``lgkmcnt(N)`` retires every LDS operation older than
the N most recent ones.  The walk is linear within each basic block; no read
issued from inline asm may be outstanding at the end of a block (the
compiler's own reads are tracked by the compiler across blocks; forgetting
them at a label only makes this check stricter, since older operations
retire first).  An ``lgkmcnt(N > 0)`` wait while a scalar-memory load is
outstanding (those complete out of order) is reported as well.
"""
from __future__ import annotations

import re

_REG = re.compile(r"v(\d+)$|v\[(\d+):(\d+)\]$")


def _regs(tok: str) -> set:
    m = _REG.fullmatch(tok)
    if not m:
        return set()
    if m.group(1) is not None:
        return {int(m.group(1))}
    return set(range(int(m.group(2)), int(m.group(3)) + 1))


def kernel_body(asm: str, name: str) -> list:
    i = asm.index(name + ":")
    j = asm.index(".Lfunc_end", i)
    return asm[i:j].split("\n")


def check(lines: list) -> tuple:
    """(number of LDS reads seen, list of problem descriptions)."""
    problems, reads = [], 0
    pend = []  # outstanding lgkm operations, oldest first: (kind, dst regs, line)
    in_asm = False
    for n, raw in enumerate(lines):
        if ";;#ASMSTART" in raw:
            in_asm = True
        elif ";;#ASMEND" in raw:
            in_asm = False
        t = raw.split(";")[0].strip()
        if not t:
            continue
        if t.endswith(":"):
            if any(k == "asm" for k, _, _ in pend):
                problems.append(f"asm LDS read outstanding at the end of the block before {t}")
            pend = []
            continue
        if t.startswith("."):
            continue
        op = t.split()[0]
        args = [a.strip().split()[0] for a in t[len(op):].split(",") if a.strip()]
        if op == "s_waitcnt":
            m = re.search(r"lgkmcnt\((\d+)\)", t)
            if m or re.fullmatch(r"s_waitcnt\s+0", t):
                lim = int(m.group(1)) if m else 0
                if lim > 0 and any(k == "smem" for k, _, _ in pend):
                    problems.append(f"line {n}: lgkmcnt({lim}) with a scalar load outstanding")
                while len(pend) > lim:
                    pend.pop(0)
            continue
        store = op.startswith(("ds_write", "global_store", "buffer_store", "scratch_store"))
        has_dst = (op.startswith(("v_", "ds_read", "ds_bpermute", "global_load", "buffer_load", "scratch_load"))
                   and not store and not op.startswith("v_cmp"))
        dst = _regs(args[0]) if has_dst and args else set()
        srcs = set()
        for a in (args[1:] if has_dst else args):
            srcs |= _regs(a)
        for kind, d, ln in pend:
            if kind in ("lds", "asm") and d and (d & srcs or d & dst):
                problems.append(f"line {n}: '{t}' touches the registers of the LDS read at line {ln}")
        if op.startswith("ds_"):
            kind = "asm" if in_asm else "lds"
            pend.append((kind, dst if (op.startswith("ds_read") or op.startswith("ds_bpermute")) else set(), n))
            reads += op.startswith("ds_read")
        elif op.startswith(("s_load", "s_buffer_load", "s_memtime", "s_memrealtime")):
            pend.append(("smem", set(), n))
    return reads, problems
