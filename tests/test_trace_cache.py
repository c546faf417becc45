"""The tile-map cache and the host tracer's threads (CPU only).

A mask function is keyed by what it computes -- code, defaults, closure
contents, the values of the globals it names -- so a new but identical lambda
per call finds the map already traced, while any change to a value it reads
traces again (the reference bakes mask_fn in when jax traces the call).  The
threaded tracer must give the same map as one thread, array for array.
"""
import numpy as np
import pytest

from jaxmodules_amd import attention as A
from jaxmodules_amd import blockmap as bm

SHAPE = (1, 300, 2, 64)
OFFSET = 3


def _make(window):
    return lambda h, q, k: (q >= k) & (q - k <= window)


def _call(mask_fn, **kw):
    return A.trace_call(SHAPE, SHAPE, SHAPE, mask_fn=mask_fn, block_size=64, **kw)[1]


def test_identical_lambdas_share_one_traced_map():
    """The same lambda expression evaluated per call (a new function object
    each time, as in a training step) traces once."""
    A.clear_cache()
    maps = [_call(lambda h, q, k: q >= k + h) for _ in range(3)]
    assert maps[0] is maps[1] is maps[2]
    assert _call(_make(40)) is _call(_make(40))


def test_a_changed_closure_value_traces_again():
    A.clear_cache()
    a, b = _call(_make(40)), _call(_make(90))
    assert a is not b and a.pairs != b.pairs


def test_a_changed_global_traces_again():
    global OFFSET
    A.clear_cache()
    fn = lambda h, q, k: q + OFFSET >= k
    a = _call(fn)
    old = OFFSET
    try:
        OFFSET = 50
        b = _call(fn)
    finally:
        OFFSET = old
    assert a is not b and b.pairs > a.pairs
    assert _call(fn) is a


def test_an_array_changed_in_place_traces_again():
    A.clear_cache()
    tiles = np.ones((2, 5, 5), bool)
    fn = lambda h, q, k: tiles[h, q // 64, k // 64]
    a = _call(fn)
    tiles[1, 2, 3] = False
    b = _call(fn)
    assert a is not b and b.pairs == a.pairs - 64 * 64


def test_a_value_it_cannot_describe_keys_by_identity():
    class Doc:
        def ids(self, x):
            return x // 100

    d = Doc()
    fn = lambda h, q, k: d.ids(q) == d.ids(k)
    assert A._mask_key(fn) is fn
    A.clear_cache()
    assert _call(fn) is _call(fn)


@pytest.mark.parametrize("name", ["per_head_tiles", "documents", "ragged_window"])
def test_threads_give_the_same_map(name, monkeypatch):
    rng = np.random.default_rng(5)
    tiles = rng.random((4, 8, 8)) < 0.4
    fns = {
        "per_head_tiles": (lambda h, q, k: tiles[h, q // 128, k // 128] & (q >= k), (1, 1000, 4, 64)),
        "documents": (lambda b, h, q, k: (q // (70 + 13 * b)) == (k // (70 + 13 * b)), (2, 900, 2, 64)),
        "ragged_window": (lambda h, q, k: abs(q - k) <= 150 + 40 * h, (1, 777, 3, 64)),
    }
    fn, shape = fns[name]
    plan = bm.make_plan(shape, shape, shape, mask_fn=fn, block_size=128)
    maps = {}
    for threads in (1, 4):
        monkeypatch.setattr(bm, "TRACE_THREADS", threads)
        maps[threads] = bm.trace(plan)
    a, b = maps[1], maps[4]
    for f in ("row_ptr", "row_ent", "col_ptr", "col_ent", "col_row", "kv_desc", "row_bits", "col_bits",
              "q_order", "kv_order"):
        assert np.array_equal(getattr(a, f), getattr(b, f)), f
    assert (a.pairs, a.n_full, a.n_partial) == (b.pairs, b.n_full, b.n_partial)


def test_a_changed_module_attribute_traces_again():
    """A mask reading a module attribute (cfg.W) is keyed by that attribute's
    value, not by the module's name."""
    import types

    cfg = types.ModuleType("mask_cfg")
    cfg.W = 100
    A.clear_cache()
    fn = lambda h, q, k: (q - k >= 0) & (q - k < cfg.W)  # noqa: E731
    a = _call(fn)
    cfg.W = 200
    b = _call(fn)
    assert a is not b and b.pairs > a.pairs
    assert b.pairs == _call(lambda h, q, k: (q - k >= 0) & (q - k < 200)).pairs


def test_numpy_functions_keep_content_keys():
    """Masks calling numpy functions (np.where, ufuncs, dtypes) are still keyed by
    content: a new identical lambda finds the traced map."""
    A.clear_cache()
    maps = [_call(lambda h, q, k: np.where(np.abs(q - k) < 30, True, np.int32(k) <= q)) for _ in range(2)]
    assert maps[0] is maps[1]
