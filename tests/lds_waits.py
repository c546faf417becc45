"""Static check of compiled kernel assembly (gfx950): no instruction reads or
overwrites the destination VGPRs of an LDS read before an ``s_waitcnt lgkmcnt``
has covered that read.

The forward, dK/dV and dQ kernels issue their MFMA operand reads as
inline-asm ``ds_read`` instructions with hand-counted waits (the compiler does not track them), so
the waits are checked on the code the compiler actually emitted.  LDS reads
complete in order, so ``lgkmcnt(N)`` retires every LDS operation older than
the N most recent ones.  The walk follows the code in layout order: the
outstanding reads at a forward branch travel to its target label, where they
merge with the fall-through path (the code after a label is walked once for
each distinct list of outstanding reads that reaches it).  No read issued from
inline asm may be outstanding at a backward branch (a loop's back edge), so
a loop header needs only the state of the path that enters it; the compiler's
own reads pending at a back edge are then not tracked into the loop, which
hides no newer read (older operations retire first).
An ``lgkmcnt(N > 0)`` wait while a scalar-memory load is outstanding (those
complete out of order) is reported as well.
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
    # the possible lists of outstanding lgkm operations (one per path that
    # reaches this point), each oldest first: (kind, dst regs, line)
    states = [[]]
    in_asm = False
    fwd = {}       # label -> state lists of the branches that jump to it
    seen = set()   # labels already passed (a branch to one of them is a back edge)
    reachable = True  # does control fall through to the next line?

    def uniq(sts):
        out, keys = [], set()
        for st in sts:
            key = tuple((k, tuple(sorted(d)), ln) for k, d, ln in st)
            if key not in keys:
                keys.add(key)
                out.append(st)
        return out

    for n, raw in enumerate(lines):
        if ";;#ASMSTART" in raw:
            in_asm = True
        elif ";;#ASMEND" in raw:
            in_asm = False
        t = raw.split(";")[0].strip()
        if not t:
            continue
        if t.endswith(":"):
            label = t[:-1]
            incoming = fwd.pop(label, [])
            if reachable:
                incoming += states
            states = uniq(incoming) or [[]]
            seen.add(label)
            reachable = True
            continue
        if t.startswith("."):
            continue
        op = t.split()[0]
        args = [a.strip().split()[0] for a in t[len(op):].split(",") if a.strip()]
        if op.startswith(("s_branch", "s_cbranch")):
            target = args[0] if args else ""
            if target in seen:
                if any(k == "asm" for st in states for k, _, _ in st):
                    problems.append(f"line {n}: asm LDS read outstanding at the back edge to {target}")
            else:
                fwd.setdefault(target, []).extend([list(st) for st in states])
            if op.startswith("s_branch"):
                reachable = False
            continue
        if op in ("s_endpgm", "s_setpc_b64"):
            if any(k == "asm" for st in states for k, _, _ in st):
                problems.append(f"line {n}: asm LDS read outstanding at {op}")
            reachable = False
            continue
        if op == "s_waitcnt":
            m = re.search(r"lgkmcnt\((\d+)\)", t)
            if m or re.fullmatch(r"s_waitcnt\s+0", t):
                lim = int(m.group(1)) if m else 0
                for st in states:
                    if lim > 0 and any(k == "smem" for k, _, _ in st):
                        problems.append(f"line {n}: lgkmcnt({lim}) with a scalar load outstanding")
                    while len(st) > lim:
                        st.pop(0)
            continue
        store = op.startswith(("ds_write", "global_store", "buffer_store", "scratch_store"))
        has_dst = (op.startswith(("v_", "ds_read", "ds_bpermute", "global_load", "buffer_load", "scratch_load"))
                   and not store and not op.startswith("v_cmp"))
        dst = _regs(args[0]) if has_dst and args else set()
        srcs = set()
        for a in (args[1:] if has_dst else args):
            srcs |= _regs(a)
        for st in states:
            for kind, d, ln in st:
                if kind in ("lds", "asm") and d and (d & srcs or d & dst):
                    problems.append(f"line {n}: '{t}' touches the registers of the LDS read at line {ln}")
        if op.startswith("ds_"):
            kind = "asm" if in_asm else "lds"
            for st in states:
                st.append((kind, dst if (op.startswith("ds_read") or op.startswith("ds_bpermute")) else set(), n))
            reads += op.startswith("ds_read")
        elif op.startswith(("s_load", "s_buffer_load", "s_memtime", "s_memrealtime")):
            for st in states:
                st.append(("smem", set(), n))
    for label in fwd:
        problems.append(f"branch to {label}, which is not in the walked code")
    return reads, sorted(set(problems), key=problems.index)
