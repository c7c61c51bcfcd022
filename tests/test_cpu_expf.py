"""The device exp (s2::expf_glibc) against the C library's expf, on the CPU.

Rust's f32::exp (the reference's softmax, sampling.rs:202-225, and SwiGLU
sigmoids, slow_ar.rs:1215-1232 / fast_ar.rs:472-485) calls glibc's expf, so
the device routine must reproduce its bits, not merely be accurate.  The
routine is compiled for the host too (s2hip_expf_host, no GPU needed); the
same source runs on the device (tests/test_gpu_ops.py checks those bits).
"""

import numpy as np
import pytest

from oracle import oracle as O
from s2hip.engine import expf_host


def _bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def _floats(u32):
    return np.ascontiguousarray(u32, np.uint32).view(np.float32)


def test_oracle_expf_is_an_accurate_exp():
    # pin the oracle's expf itself: within 0.51 ulp of exp in float64 over
    # [-104, 89], exact at 0, +-inf and NaN handling as IEEE exp
    x = np.linspace(-103.9, 88.7, 2_000_001, dtype=np.float32)
    y = O.expf(x)
    ref = np.exp(x.astype(np.float64))
    ulp = np.spacing(ref.astype(np.float32)).astype(np.float64)
    err = np.abs(y.astype(np.float64) - ref) / ulp
    assert err.max() <= 0.51
    sp = O.expf(np.array([0.0, -0.0, np.inf, -np.inf, np.nan, 89.0, -110.0], np.float32))
    assert sp[0] == 1.0 and sp[1] == 1.0 and sp[2] == np.inf and sp[3] == 0.0
    assert np.isnan(sp[4]) and sp[5] == np.inf and sp[6] == 0.0


@pytest.mark.parametrize("start", [0, 29])
def test_expf_glibc_bits_strided_over_every_float(start):
    # every 59th bit pattern from `start`: ~73 M inputs per case, all binades,
    # both signs, subnormal results, overflow, infinities and NaNs
    for lo in range(start, 1 << 32, 59 << 24):
        u = np.arange(lo, min(lo + (59 << 24), 1 << 32), 59, dtype=np.uint64).astype(np.uint32)
        x = _floats(u)
        got, ref = expf_host(x), O.expf(x)
        same = (_bits(got) == _bits(ref)) | (np.isnan(got) & np.isnan(ref))
        assert same.all(), x[~same][:5]


def test_expf_glibc_bits_on_softmax_arguments():
    # the sampler's arguments (v - max) / T lie in [-inf, 0]: dense there
    rng = np.random.default_rng(5)
    x = np.concatenate([
        -rng.exponential(3.0, 4_000_000).astype(np.float32),
        -rng.uniform(0, 104, 4_000_000).astype(np.float32),
        _floats(np.arange(0xBF800000, 0xBF800000 + 2_000_000, dtype=np.uint32)),  # just below -1
        _floats(np.arange(0x80000000, 0x80000000 + 2_000_000, dtype=np.uint32)),  # -0 and tiny negatives
    ])
    assert (_bits(expf_host(x)) == _bits(O.expf(x))).all()


def test_a_correctly_rounded_exp_would_fail_this_check():
    # the point of the routine: rounding exp computed in double does not
    # reproduce glibc on this range, so the bit test above has teeth
    x = -rng_uniform(3_000_000)
    cr = np.exp(x.astype(np.float64)).astype(np.float32)
    assert (_bits(cr) != _bits(O.expf(x))).sum() > 100
    assert (_bits(expf_host(x)) == _bits(O.expf(x))).all()


def rng_uniform(n):
    return np.random.default_rng(9).uniform(0, 17, n).astype(np.float32)
