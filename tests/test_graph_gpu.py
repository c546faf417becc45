"""HIP graph capture of one forward + backward step through the C ABI.

mattn_fwd and the three mattn_bwd_stage calls issue kernel launches only (no
allocation, no memset, no host synchronisation), so a caller can capture a
whole training step into a HIP graph (torch.cuda.CUDAGraph here) and replay
it, as launch-bound loops do.  The graph is replayed several times, with the
program's own eager work (the outputs overwritten, an eager step) and
synchronisations between the replays, and every replay must reproduce the
eager step bit for bit (the kernels are deterministic: no atomics).  Cases:
D = 128 with the stored dS and the split-row kernels, D = 64 with the
split-row passes inside the main kernels, and the reference benchmark's
residue-class mask at D = 64."""
import ctypes
import math

import pytest

torch = pytest.importorskip("torch")

pytestmark = pytest.mark.gpu


class _Step:
    """One problem's buffers and its fwd + bwd launches on a given stream."""

    def __init__(self, d, L, kw, dtype=torch.bfloat16, B=1, Hq=4, Hkv=2, scaled=False):
        from jaxmodules_amd import _lib
        from jaxmodules_amd import attention as A

        self._lib, self.lib = _lib, _lib.load()
        dev = torch.device("cuda:0")
        g = torch.Generator(device=dev)
        g.manual_seed(11)
        f = d ** -0.25 if scaled else 1.0
        self.q = (torch.randn((B, L, Hq, d), generator=g, device=dev) * f).to(dtype)
        self.k = (torch.randn((B, L, Hkv, d), generator=g, device=dev) * f).to(dtype)
        self.v = (torch.randn((B, L, Hkv, d), generator=g, device=dev) * f).to(dtype)
        self.do = torch.randn((B, L, Hq, d), generator=g, device=dev)
        self.o = torch.empty((B, L, Hq, d), dtype=torch.float32, device=dev)
        self.lse = torch.empty((B, Hq, L), dtype=torch.float32, device=dev)
        self.dq, self.dk, self.dv = (torch.empty_like(x) for x in (self.q, self.k, self.v))
        _, tm = A.trace_call(tuple(self.q.shape), tuple(self.k.shape), tuple(self.v.shape), device=dev, **kw)
        self.p = A._problem(self.q, self.k, self.v, self.o, 1.0 / math.sqrt(d), do=self.do, dq=self.dq,
                            dk=self.dk, dv=self.dv)
        self.p.flags = _lib.MATTN_FWD_FOR_BWD
        self.bm = A.device_blockmap(tm, dev)
        self.p.flags = A.bwd_flags(self.p, self.bm)
        self.stored_ds = bool(self.p.flags & _lib.MATTN_BWD_DS)
        nws = int(self.lib.mattn_bwd_workspace_bytes(ctypes.byref(self.p), ctypes.byref(self.bm)))
        self.ws = torch.empty(nws + 256, dtype=torch.uint8, device=dev)
        self.wptr, self.ws_bytes = (self.ws.data_ptr() + 255) & ~255, nws
        nres = int(self.lib.mattn_fwd_workspace_bytes(ctypes.byref(self.p)))
        self.res = torch.empty(nres + 256, dtype=torch.uint8, device=dev)
        self.rptr = (self.res.data_ptr() + 255) & ~255

    def outputs(self):
        return (self.o, self.lse, self.dq, self.dk, self.dv)

    def run(self, stream):
        lib, chk = self.lib, self._lib.check
        chk(lib.mattn_fwd(ctypes.byref(self.p), ctypes.byref(self.bm), self.q.data_ptr(), self.k.data_ptr(),
                          self.v.data_ptr(), self.o.data_ptr(), self.lse.data_ptr(), self.rptr, stream), "fwd")
        for s in range(3):
            chk(lib.mattn_bwd_stage(ctypes.byref(self.p), ctypes.byref(self.bm), s, self.q.data_ptr(),
                                    self.k.data_ptr(), self.v.data_ptr(), self.o.data_ptr(), self.do.data_ptr(),
                                    self.lse.data_ptr(), self.rptr, self.wptr, self.ws_bytes, self.dq.data_ptr(),
                                    self.dk.data_ptr(), self.dv.data_ptr(), stream), f"bwd stage {s}")


def _cases():
    from jaxmodules_amd import masks

    return {
        "d128_causal": (128, 640, dict(is_causal=True), False),
        "d64_causal_unit": (64, 640, dict(is_causal=True), False),
        "d64_residue": (64, 1024, dict(mask_fn=masks.intersect(masks.same_residue(8), masks.causal())), False),
    }


@pytest.mark.parametrize("case", ["d128_causal", "d64_causal_unit", "d64_residue"])
def test_graph_replays_equal_the_eager_step(case):
    d, L, kw, scaled = _cases()[case]
    print(f"[graph] {case}", flush=True)
    st = _Step(d, L, kw, scaled=scaled)
    if d == 128:
        assert st.stored_ds  # the default D = 128 backward: dS stored, then the split kernels
    cur = torch.cuda.current_stream()
    st.run(cur.cuda_stream)
    torch.cuda.synchronize()
    want = [x.clone() for x in st.outputs()]
    assert all(torch.isfinite(x).all() for x in want)

    # capture (after a warm-up step on the capture's side stream, as torch asks)
    side = torch.cuda.Stream()
    side.wait_stream(cur)
    with torch.cuda.stream(side):
        st.run(side.cuda_stream)
    cur.wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        st.run(torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()

    for r in range(4):
        for x in st.outputs():  # eager work between replays: the outputs overwritten
            x.fill_(float("nan"))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        for name, a, b in zip(("O", "lse", "dQ", "dK", "dV"), st.outputs(), want):
            assert torch.equal(a, b), f"replay {r}: {name} differs from the eager step"
        if r == 1:  # an eager step in between
            st.run(cur.cuda_stream)
            torch.cuda.synchronize()
            for name, a, b in zip(("O", "lse", "dQ", "dK", "dV"), st.outputs(), want):
                assert torch.equal(a, b), f"eager step after replay {r}: {name} differs"
    print(f"[graph] {case}: 4 replays equal the eager step", flush=True)
