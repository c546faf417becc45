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
Scalar-memory loads share the counter but complete out of order: an
``lgkmcnt(N)`` only guarantees that at most N operations are outstanding,
which may all be LDS reads, so it retires every LDS operation older than the
N most recent LDS operations (scalar loads not counted), and retires scalar
loads only at N = 0.

``check_dma`` checks the other counter: every global->LDS load (the ``lds``
forms of ``global_load`` / ``buffer_load``) must have retired at the next
``s_barrier``, which is where the double-buffered kernels hand a filled LDS
buffer to the other waves.  Vector memory operations (loads and, on gfx9,
stores) retire in issue order, so ``vmcnt(N)`` retires all but the N most
recent.  Loads legitimately stay in flight across a loop's back edge (the
prefetch of the next iteration), so there the walk is repeated with the back
edges' states added at the loop header until no new state reaches it.
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
                for i, st in enumerate(states):
                    if lim == 0:
                        st.clear()
                        continue
                    keep = [e for e in st if e[0] != "smem"][-lim:]
                    states[i] = [e for e in st if e[0] == "smem" or any(e is x for x in keep)]
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


_VMEM = ("global_load", "global_store", "global_atomic", "buffer_load", "buffer_store", "buffer_atomic",
         "flat_", "scratch_")


def _fold(st: tuple, keep: int) -> tuple:
    """A state with at most `keep` tracked operations: the older ones fold into
    one leading ("old", line) entry when any of them is a global->LDS load.
    Exact for this walk, since no wait in the kernel keeps more than `keep`
    operations outstanding: the next vmcnt retires every folded operation."""
    if len(st) <= keep:
        return st
    old = [e for e in st[:len(st) - keep] if e[0] in ("dma", "old")]
    rest = st[len(st) - keep:] if keep else ()
    return ((("old", old[0][1]),) if old else ()) + rest


def _dma_walk(lines: list, loop_in: dict, keep: int = 0) -> tuple:
    """One layout-order walk for check_dma: (problems, back-edge states by label)."""
    problems = []
    states = [()]
    fwd, seen, back = {}, set(), {}
    reachable = True
    for n, raw in enumerate(lines):
        t = raw.split(";")[0].strip()
        if not t:
            continue
        if t.endswith(":"):
            label = t[:-1]
            incoming = fwd.pop(label, []) + list(loop_in.get(label, ()))
            if reachable:
                incoming += states
            states = list(dict.fromkeys(incoming)) or [()]
            seen.add(label)
            reachable = True
            continue
        if t.startswith("."):
            continue
        op = t.split()[0]
        if op.startswith(("s_branch", "s_cbranch")):
            target = t[len(op):].strip().split()[0] if t[len(op):].strip() else ""
            if target in seen:
                back.setdefault(target, set()).update(states)
            else:
                fwd.setdefault(target, []).extend(states)
            if op.startswith("s_branch"):
                reachable = False
            continue
        if op in ("s_endpgm", "s_setpc_b64"):
            reachable = False
            continue
        if op == "s_waitcnt":
            m = re.search(r"vmcnt\((\d+)\)", t)
            if m or re.fullmatch(r"s_waitcnt\s+0", t):
                lim = int(m.group(1)) if m else 0
                states = [st[max(0, len(st) - lim):] if lim else () for st in states]
            continue
        if op == "s_barrier":
            if "lds-only" in raw:  # a barrier that hands no DMA-filled buffer over (marked in the source)
                continue
            for st in states:
                for kind, ln in st:
                    if kind in ("dma", "old"):
                        problems.append(f"line {n}: s_barrier with the global->LDS load of line {ln} outstanding")
            continue
        if op.startswith(_VMEM):
            kind = "dma" if re.search(r"\blds\b", t[len(op):]) or op.endswith("_lds_dwordx4") else "vmem"
            states = list(dict.fromkeys(_fold(st + ((kind, n),), keep) for st in states))
    for label in fwd:
        problems.append(f"branch to {label}, which is not in the walked code")
    return problems, back


def check_dma(lines: list, max_rounds: int = 20) -> tuple:
    """(number of global->LDS loads seen, list of problem descriptions)."""
    dma = sum(1 for l in lines if re.search(r"^\s*(global_load_lds_\w+|buffer_load_\w+.*\blds\b)", l.split(";")[0]))
    # the largest vmcnt any wait keeps outstanding bounds what a state must track
    keep = max([int(m) for l in lines for m in re.findall(r"vmcnt\((\d+)\)", l.split(";")[0])] + [0])
    loop_in: dict = {}
    for _ in range(max_rounds):
        problems, back = _dma_walk(lines, loop_in, keep)
        grown = False
        for label, sts in back.items():
            cur = loop_in.setdefault(label, set())
            if not sts <= cur:
                cur |= sts
                grown = True
        if not grown:
            return dma, sorted(set(problems), key=problems.index)
    return dma, ["the loop states did not settle"]
