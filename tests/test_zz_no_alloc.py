"""fh_sample_logits_noalloc against fh_sample_logits, through the C ABI.

The no-allocation entry point keeps its scratch in one fixed device array shared by
every call on the device, so it is checked on consecutive calls, each following
call with a smaller vocabulary and a shorter history than the one before (a stale
tail of the previous call's scratch must not leak into the draw), across the
sampler's options (greedy, temperature, top-k, repetition penalty, n-gram bans)
and both sampler kernels (V <= 16384 and above).  Bar: the ids are equal.
"""
import ctypes

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _draw(fhp, fn, be, dev, V, hist, T, k, u, pen, ng):
    N = fhp._native
    h = np.ascontiguousarray(hist, np.int32)
    opts = N.Sampling(float(T), int(k), float(pen), int(ng), -1, 0)
    out = ctypes.c_int32(-7)
    ptr = dev.ptr if isinstance(dev.ptr, ctypes.c_void_p) else ctypes.c_void_p(dev.ptr)
    N.check(fn(be.handle, ptr, V, h.ctypes.data if h.size else None, h.size,
               ctypes.byref(opts), float(u), ctypes.byref(out)))
    return out.value


@pytest.mark.parametrize("first_V,second_V", [(16384, 2256), (65536, 30000), (30000, 100)])
def test_noalloc_sampler_matches_allocating_sampler(fhp, first_V, second_V):
    N = fhp._native
    lib = N.lib()
    be = fhp.HipBackend(0)  # calls only the no-allocation entry point
    ref = fhp.HipBackend(0)  # the allocating sampler, on a context of its own
    rng = np.random.default_rng(first_V + second_V)
    opts = [(0.0, 0, 1.0, 0), (0.7, 30, 1.1, 4), (1.0, 0, 2.0, 1), (0.9, 1, 1.0, 2), (0.8, 5000, 1.3, 3)]
    for T, k, pen, ng in opts:
        for V, n_hist in ((first_V, 900), (second_V, 40)):  # the second call is smaller in both
            lg = (rng.standard_normal(V) * 2).astype(np.float32)
            lg[rng.integers(0, V, 8)] = lg.max()  # ties at the top
            hist = rng.integers(0, min(V, 60), size=n_hist).astype(np.int32)
            u = float(rng.random())
            dev = fhp.DeviceBuffer.from_array(be, lg)
            want = _draw(fhp, lib.fh_sample_logits, ref, dev, V, hist, T, k, u, pen, ng)
            got = _draw(fhp, lib.fh_sample_logits_noalloc, be, dev, V, hist, T, k, u, pen, ng)
            dev.free()
            assert got == want, (V, n_hist, T, k, pen, ng, got, want)
            assert 0 <= got < V
    # the no-allocation calls never used the context's own (allocated) scratch
    assert be.memory()[1] == 0 and ref.memory()[1] > 0
    be.dispose()
    ref.dispose()


def test_noalloc_sampler_allocates_nothing(fhp):
    # a fresh context that only ever calls the no-allocation entry point: after one
    # warm-up call (which loads the library's kernels), calls at the largest sizes and
    # smaller ones leave the device's free memory and the context's scratch unchanged
    lib = fhp._native.lib()
    be = fhp.HipBackend(0)
    rng = np.random.default_rng(5)
    rows = {V: fhp.DeviceBuffer.from_array(be, (rng.standard_normal(V) * 2).astype(np.float32))
            for V in (65536, 16384, 100)}
    _draw(fhp, lib.fh_sample_logits_noalloc, be, rows[100], 100, [1, 2], 0.7, 5, 0.3, 1.1, 2)
    free0, scr0 = be.memory()
    for V, n_hist in ((65536, 32768), (100, 10), (16384, 5000), (65536, 32768), (16384, 0)):
        hist = rng.integers(0, V, size=n_hist).astype(np.int32)
        for T, k, pen, ng in ((0.0, 0, 1.0, 0), (0.8, 40, 1.2, 3)):
            got = _draw(fhp, lib.fh_sample_logits_noalloc, be, rows[V], V, hist, T, k, float(rng.random()), pen, ng)
            assert 0 <= got < V
    free1, scr1 = be.memory()
    assert scr0 == 0 and scr1 == 0
    assert free1 == free0, (free0, free1)
    for b in rows.values():
        b.free()
    be.dispose()


def test_noalloc_sampler_rejects_sizes_beyond_its_scratch(fhp):
    N = fhp._native
    lib = N.lib()
    be = fhp.HipBackend(0)
    dev = fhp.DeviceBuffer.from_array(be, np.zeros(16, np.float32))
    with pytest.raises(fhp.HipError, match="no-allocation scratch"):
        _draw(fhp, lib.fh_sample_logits_noalloc, be, dev, 16, np.zeros(32769, np.int32), 0.7, 0, 0.5, 1.0, 0)
    dev.free()
    be.dispose()
