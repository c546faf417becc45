"""The hand-counted LDS waits of the forward, dK/dV and dQ kernels, and the
vmcnt waits that must retire their global->LDS loads before each barrier,
checked on their compiled gfx950 assembly (no GPU needed: hipcc
cross-compiles here)."""
import os
import re
import shutil

import pytest

from jaxmodules_amd import build as B

from tests import lds_waits

pytestmark = pytest.mark.skipif(not (shutil.which("hipcc") or os.path.exists("/opt/rocm/bin/hipcc")),
                                reason="hipcc not available")


def _asm(src_name, tmp_path_factory):
    """The source compiled to gfx950 assembly with the library's own flags."""
    src = os.path.join(B.CSRC, src_name)
    out = str(tmp_path_factory.mktemp("asm") / (src_name + ".s"))
    sched = B.SCHED.get(src_name)
    flags = B.common_flags() + (["-mllvm", f"-amdgpu-sched-strategy={sched}"] if sched else [])
    B._run([B.hipcc(), *flags, "--cuda-device-only", "-S", src, "-o", out])
    return open(out).read()


@pytest.fixture(scope="module")
def dkdv_asm(tmp_path_factory):
    return _asm("bwd_dkdv.hip", tmp_path_factory)


@pytest.fixture(scope="module")
def dq_asm(tmp_path_factory):
    return _asm("bwd_dq.hip", tmp_path_factory)


@pytest.fixture(scope="module")
def fwd_asm(tmp_path_factory):
    return _asm("fwd.hip", tmp_path_factory)


def _kernels(asm, stem="13bwd_dkdv_mfma"):
    return sorted(set(re.findall(rf"^(_ZN5mattn{stem}\w+):", asm, re.M)))


@pytest.mark.parametrize("which", ["dkdv", "dq", "dq_ds", "fwd"])
def test_every_instantiation_waits_before_use(which, dkdv_asm, dq_asm, fwd_asm):
    asm, stem, least, count = {
        # D = 64 / 128 x bfloat16 / float16 x (storing dS, not storing it), and the split
        # kernel at D = 128 (at D = 64 the first kernel corrects the split columns itself)
        "dkdv": (dkdv_asm, "13bwd_dkdv_mfma", 60, 10),
        # D = 64 / 128 x bfloat16 / float16 x (other tiles, split tiles); at D = 64 the
        # first also serves the split tiles when dS is not stored
        "dq": (dq_asm, "11bwd_dq_mfma", 60, 8),
        "dq_ds": (dq_asm, "9bwd_dq_ds", 40, 4),
        # ... x float32 / 16-bit output x (main, split tiles at D = 128; at D = 64 the main
        # kernel walks its split rows again itself)
        "fwd": (fwd_asm, "8fwd_mfma", 50, 12),
    }[which]
    names = _kernels(asm, stem)
    assert len(names) == count, names
    for name in names:
        reads, problems = lds_waits.check(lds_waits.kernel_body(asm, name))
        assert reads > least, (name, reads)
        assert not problems, (name, problems[:5])


def test_checker_flags_a_missing_wait(dkdv_asm):
    """Removing one of the hand-counted waits must be reported."""
    name = _kernels(dkdv_asm)[0]
    body = lds_waits.kernel_body(dkdv_asm, name)
    k = next(i for i, l in enumerate(body) if "s_waitcnt lgkmcnt(4)" in l)
    planted = body[:k] + ["\ts_nop 0"] + body[k + 1:]
    _, problems = lds_waits.check(planted)
    assert problems


_BRANCHY = """\
;;#ASMSTART
\tds_read_b128 v[4:7], v1 offset:0
;;#ASMEND
\ts_cbranch_scc1 .LBB0_2
\tv_mov_b32_e32 v9, 0
\ts_waitcnt lgkmcnt(0)
.LBB0_2:
\tv_add_f32_e32 v8, v4, v8
\ts_endpgm
"""


def test_checker_follows_forward_branches():
    """A read still outstanding on the branch path reaches the label: using its
    registers there is reported even though the fall-through path waited."""
    _, problems = lds_waits.check(_BRANCHY.split("\n"))
    assert any("touches the registers" in p for p in problems)
    fixed = _BRANCHY.replace(".LBB0_2:\n", ".LBB0_2:\n\ts_waitcnt lgkmcnt(0)\n")
    assert lds_waits.check(fixed.split("\n"))[1] == []


@pytest.mark.parametrize("which", ["dkdv", "dq", "dq_ds", "fwd"])
def test_every_instantiation_retires_its_lds_dma_before_each_barrier(which, dkdv_asm, dq_asm, fwd_asm):
    asm, stem, least, count = {
        "dkdv": (dkdv_asm, "13bwd_dkdv_mfma", 6, 10),
        "dq": (dq_asm, "11bwd_dq_mfma", 10, 8),
        "dq_ds": (dq_asm, "9bwd_dq_ds", 6, 4),      # D = 64: 2 K' loads x (prologue + 2 unrolled steps)
        "fwd": (fwd_asm, "8fwd_mfma", 10, 12),
    }[which]
    names = _kernels(asm, stem)
    assert len(names) == count, names
    for name in names:
        dma, problems = lds_waits.check_dma(lds_waits.kernel_body(asm, name))
        assert dma >= least, (name, dma)
        assert not problems, (name, problems[:5])


def test_dma_checker_flags_a_dq_ds_wait_that_leaves_a_dma_in_flight(dq_asm):
    """A dQ wave's last loads before the next iteration's wait are the DMA of
    the next sub-block's K' rows and dS~ blocks; vmcnt(4) there leaves the
    newest of them outstanding at the barrier: reported."""
    name = _kernels(dq_asm, "9bwd_dq_ds")[0]
    body = lds_waits.kernel_body(dq_asm, name)
    waits = [i for i, l in enumerate(body) if l.strip() == "s_waitcnt vmcnt(0)"]
    assert waits
    planted = [("\ts_waitcnt vmcnt(4)" if i in waits else l) for i, l in enumerate(body)]
    _, problems = lds_waits.check_dma(planted)
    assert any("global->LDS load" in p for p in problems)


_LOOP = """\
\tglobal_load_lds_dwordx4 v1, s[0:1]
\tglobal_load_dwordx4 v[4:7], v[2:3], off
\tglobal_load_dwordx4 v[8:11], v[2:3], off
.LBB0_1:
\ts_waitcnt vmcnt(2)
\ts_barrier
\tglobal_load_lds_dwordx4 v1, s[0:1]
\tglobal_load_dwordx4 v[4:7], v[2:3], off
\ts_cbranch_scc1 .LBB0_1
\ts_waitcnt vmcnt(0)
\ts_endpgm
"""


def test_dma_checker_carries_loads_across_the_back_edge():
    """On entry two loads follow the DMA, so vmcnt(2) retires it; around the
    loop only one does, and the same wait leaves the loop's DMA outstanding."""
    _, problems = lds_waits.check_dma(_LOOP.split("\n"))
    assert problems and all("load of line 6 outstanding" in p for p in problems), problems
    fixed = _LOOP.replace("vmcnt(2)", "vmcnt(1)", 1)
    assert lds_waits.check_dma(fixed.split("\n"))[1] == []


_MARKED = """\
\tglobal_load_lds_dwordx4 v1, s[0:1]
\ts_waitcnt lgkmcnt(0)
\ts_barrier ; lds-only: global->LDS loads may be in flight
\tglobal_store_dwordx4 v[2:3], v[4:7], off
\tglobal_store_dwordx4 v[2:3], v[4:7], off
\ts_barrier
\ts_endpgm
"""


def test_dma_checker_exempts_only_marked_barriers():
    """A barrier marked lds-only (barrier_lds_dma_in_flight) may have a DMA in
    flight; the load is still tracked, through the stores that fold it away
    (no wait in the code keeps any operation outstanding), to the next,
    unmarked barrier, which is reported."""
    _, problems = lds_waits.check_dma(_MARKED.split("\n"))
    assert len(problems) == 1 and problems[0].startswith("line 5: s_barrier") and "line 0" in problems[0]
    fixed = _MARKED.replace("\ts_barrier\n\ts_endpgm", "\ts_waitcnt vmcnt(0)\n\ts_barrier\n\ts_endpgm")
    assert lds_waits.check_dma(fixed.split("\n"))[1] == []
