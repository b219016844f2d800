"""The device arithmetic source (jieyu_amd/csrc/jy_device.h), built for the host.

The helpers are __host__ __device__; oracle/Makefile compiles the same source for
x86 (oracle/_build/libjydevmath.so) so it can be checked exhaustively here against
the host libm the reference links and against the C oracle.  The GPU build of the
source is checked by the GPU parity tests, end to end.
"""
import ctypes as C
import os

import numpy as np
import pytest

from conftest import ptr

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
SO = os.path.join(ROOT, "oracle", "_build", "libjydevmath.so")


@pytest.fixture(scope="module")
def dm():
    if not os.path.exists(SO):
        pytest.fail(f"{SO} missing: run `make -C oracle`")
    lib = C.CDLL(SO)
    lib.jydm_expf_mismatches.restype = C.c_uint64
    lib.jydm_expf_mismatches.argtypes = [C.c_uint64, C.c_uint64, C.c_uint64, C.c_void_p]
    lib.jydm_expf.restype = C.c_float
    lib.jydm_expf.argtypes = [C.c_float]
    lib.jydm_silu.argtypes = [C.c_void_p, C.c_void_p, C.c_int]
    lib.jydm_half_to_float.argtypes = [C.c_void_p, C.c_void_p, C.c_int]
    lib.jydm_quant.argtypes = [C.c_void_p, C.c_int, C.c_void_p, C.c_void_p]
    return lib


def _mismatches(dm, lo, hi, step):
    first = C.c_uint32(0)
    n = dm.jydm_expf_mismatches(lo, hi, step, C.byref(first))
    return n, hex(first.value)


def test_expf_softmax_domain_exhaustive(dm):
    """Every float in [-104, -0] -- all the softmax feeds expf (x - max <= 0) before it
    underflows -- gives glibc's expf bits."""
    lo = 0x80000000
    hi = int(np.array([-104.0], np.float32).view(np.uint32)[0]) + 1
    assert _mismatches(dm, lo, hi, 1) == (0, "0x0")


def test_expf_whole_range_exhaustive(dm):
    """All 2^32 patterns (positive, overflow, subnormal, NaN and inf included)."""
    assert _mismatches(dm, 0, 1 << 32, 1) == (0, "0x0")


def test_expf_special_values(dm):
    assert dm.jydm_expf(0.0) == 1.0
    assert dm.jydm_expf(-0.0) == 1.0
    assert dm.jydm_expf(float("-inf")) == 0.0
    assert dm.jydm_expf(float("inf")) == float("inf")
    assert np.isnan(dm.jydm_expf(float("nan")))
    assert dm.jydm_expf(-200.0) == 0.0
    assert dm.jydm_expf(100.0) == float("inf")
    # exp(1) correctly rounded to float
    assert dm.jydm_expf(1.0) == np.float32(np.e)


def test_silu_matches_oracle_and_golden(dm, oracle_lib):
    x = np.arange(-100.0, 100.0, 0.00037, dtype=np.float64).astype(np.float32)
    x = np.concatenate([x, np.array([0.0, -0.0, 1e-38, -1e-38, 88.7, -88.7, 1e4, -1e4], np.float32)])
    a, b = np.zeros_like(x), np.zeros_like(x)
    dm.jydm_silu(ptr(x), ptr(a), x.size)
    # the oracle's SiLU takes its vector-body route for every full group of 8
    n8 = x.size // 8 * 8
    oracle_lib.jyo_silu(ptr(x[:n8].copy()), ptr(b[:n8]), n8)
    assert np.array_equal(a[:n8].view(np.uint32), b[:n8].view(np.uint32))
    kz = np.load(os.path.join(ROOT, "tests", "golden", "kernels.npz"))
    xs, ys = kz["silu_4864.x"], kz["silu_4864.y"]
    got = np.zeros_like(xs)
    dm.jydm_silu(ptr(xs), ptr(got), xs.size)
    assert np.array_equal(got.view(np.uint32), ys.view(np.uint32))


def test_half_to_float_exhaustive(dm):
    h = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16)
    got = np.zeros(h.size, np.float32)
    dm.jydm_half_to_float(ptr(h), ptr(got), h.size)
    want = h.view(np.float16).astype(np.float32)
    fin = np.isfinite(want)
    assert np.array_equal(got[fin].view(np.uint32), want[fin].view(np.uint32))
    assert np.array_equal(np.isnan(got), np.isnan(want))
    assert np.array_equal(got[np.isinf(want)], want[np.isinf(want)])


def test_quant_matches_kv_pack(dm, oracle_lib):
    rng = np.random.default_rng(2)
    for hd in (4, 64, 128):
        for scale in (1e-9, 1e-3, 1.0, 300.0):
            v = (rng.standard_normal(hd) * scale).astype(np.float32)
            if hd == 4:
                v[:] = [127 * scale, 0.5 * scale, -2.5 * scale, 3.5 * scale]
            q, s = np.zeros(hd, np.int8), np.zeros(1, np.float32)
            dm.jydm_quant(ptr(v), hd, ptr(q), ptr(s))
            q2, s2 = np.zeros(hd, np.int8), np.zeros(1, np.float32)
            oracle_lib.jyo_kv_pack(ptr(v.copy()), ptr(q2), ptr(s2), 1, hd, 1)
            assert np.array_equal(q, q2) and s.view(np.uint32)[0] == s2.view(np.uint32)[0]
