"""The allocation-free sampler entry point (s2hip_op_sample_noalloc) against
the existing one (s2hip_op_sample), through the C ABI: identical tokens and
RNG states on consecutive calls (the second with fewer logits, so stale
values left in the shared device array would show), at the 8191-logit limit,
and a clear error beyond it; the library's device-allocation count does not
move across the allocation-free calls and grows across s2hip_op_sample's."""

import ctypes

import numpy as np
import pytest

from s2hip import _lib, synth

pytestmark = pytest.mark.gpu


def _sample(L, h, fn, logits, T, top_p, top_k, always, rng):
    x = np.ascontiguousarray(logits, np.float32)
    smp = _lib.Sampler(T, top_p, top_k)
    st = ctypes.c_uint64(rng)
    tok = ctypes.c_uint32(0)
    err = ctypes.create_string_buffer(_lib.ERR_CAP)
    ok = fn(h, x.ctypes.data, x.size, ctypes.byref(smp), -1 if always is None else always, ctypes.byref(st),
            ctypes.byref(tok), err, len(err))
    return ok, tok.value, st.value, err.value.decode()


def _allocs(L):
    c = ctypes.c_uint64(0)
    L.s2hip_device_allocations(ctypes.byref(c))
    return c.value


def test_noalloc_sampler_matches_existing_entry_point(tiny_gguf):
    from s2hip import Engine

    with Engine(tiny_gguf, 64, synth.TINY.im_end_id) as e:
        L, h = e._L, e._h
        rng = np.random.default_rng(7)
        for T, top_p, top_k in [(0.7, 0.9, 0), (0.0, 1.0, 0), (1.0, 0.95, 30)]:
            for n in (8191, 4096, 37):  # consecutive calls, each smaller than the last
                logits = (rng.standard_normal(n) * 2).astype(np.float32)
                always = int(rng.integers(0, n)) if n > 100 else None
                st = int(rng.integers(1, 1 << 62))
                n0 = _allocs(L)
                a = _sample(L, h, L.s2hip_op_sample, logits, T, top_p, top_k, always, st)
                n1 = _allocs(L)
                b = _sample(L, h, L.s2hip_op_sample_noalloc, logits, T, top_p, top_k, always, st)
                assert n1 > n0 and _allocs(L) == n1, (n0, n1, _allocs(L))
                assert a[0] == 1 and b[0] == 1, (a, b)
                assert a[1:3] == b[1:3], (T, n, a, b)
        ok, _, st, msg = _sample(L, h, L.s2hip_op_sample_noalloc, np.zeros(8192, np.float32), 0.7, 0.9, 0, None, 5)
        assert ok == 0 and "at most 8191 logits" in msg and st == 5
        # still usable after the rejected call
        logits = rng.standard_normal(100).astype(np.float32)
        assert (_sample(L, h, L.s2hip_op_sample_noalloc, logits, 0.7, 0.9, 0, None, 11)[1:3] ==
                _sample(L, h, L.s2hip_op_sample, logits, 0.7, 0.9, 0, None, 11)[1:3])
