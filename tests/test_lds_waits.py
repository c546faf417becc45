"""The hand-counted LDS waits of the dK/dV kernel, checked on its compiled
gfx950 assembly (no GPU needed: hipcc cross-compiles here)."""
import os
import re
import shutil

import pytest

from jaxmodules_amd import build as B

from tests import lds_waits

pytestmark = pytest.mark.skipif(not (shutil.which("hipcc") or os.path.exists("/opt/rocm/bin/hipcc")),
                                reason="hipcc not available")


@pytest.fixture(scope="module")
def dkdv_asm(tmp_path_factory):
    src = os.path.join(B.CSRC, "bwd_dkdv.hip")
    out = str(tmp_path_factory.mktemp("asm") / "bwd_dkdv.s")
    sched = B.SCHED.get("bwd_dkdv.hip")
    flags = B.common_flags() + (["-mllvm", f"-amdgpu-sched-strategy={sched}"] if sched else [])
    B._run([B.hipcc(), *flags, "--cuda-device-only", "-S", src, "-o", out])
    return open(out).read()


def _kernels(asm):
    return sorted(set(re.findall(r"^(_ZN5mattn13bwd_dkdv_mfma\w+):", asm, re.M)))


def test_every_dkdv_instantiation_waits_before_use(dkdv_asm):
    names = _kernels(dkdv_asm)
    assert len(names) == 4, names          # D = 64 / 128 x bfloat16 / float16
    for name in names:
        reads, problems = lds_waits.check(lds_waits.kernel_body(dkdv_asm, name))
        assert reads > 100, (name, reads)
        assert not problems, (name, problems[:5])


def test_checker_flags_a_missing_wait(dkdv_asm):
    """Removing one of the hand-counted waits must be reported."""
    name = _kernels(dkdv_asm)[0]
    body = lds_waits.kernel_body(dkdv_asm, name)
    k = next(i for i, l in enumerate(body) if "s_waitcnt lgkmcnt(4)" in l)
    planted = body[:k] + ["\ts_nop 0"] + body[k + 1:]
    _, problems = lds_waits.check(planted)
    assert problems
