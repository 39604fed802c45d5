"""Brute force of the fixed-point primitives on the GPU against the oracle.

tests/prims/libprims.so evaluates the library's own device code
(llm-accel_amd/csrc/fixed_point.h, attn_common.h) over whole input
ranges: fx_recip and fx_silu over every int16, fx_rsqrt and fx_inv_sum
over every value below 2^16 and one value in each of the 65,536 2^16-wide
bands of int32 (plus the thresholds of their seeds and saturation), the
attention product term (the kernels' clamp to [-2048, 2048] plus the
saturation correction c(a) = floor((8 - a) / 16)) over every int16 of
each operand against the other operand's extremes and a sweep, and the
Q2.14 probability lookup over every score difference.  Each is compared
with the oracle's function (orc_recip, orc_rsqrt, orc_silu, orc_inv_sum,
orc_fm_wt_term, orc_attn_prob)."""
import ctypes
import os

import numpy as np
import pytest

from oracle import orc

pytestmark = pytest.mark.gpu

HERE = os.path.dirname(os.path.abspath(__file__))
P_RECIP, P_RSQRT, P_SILU, P_INV_SUM, P_TERM, P_PROB = range(6)


@pytest.fixture(scope="module")
def prims():
    path = os.path.join(HERE, "prims", "libprims.so")
    if not os.path.exists(path):
        raise RuntimeError(f"{path} is missing: build it with `make -C tests/prims`")
    lib = ctypes.CDLL(path)
    i32p = ctypes.POINTER(ctypes.c_int32)
    lib.prims_eval.restype = ctypes.c_int
    lib.prims_eval.argtypes = [ctypes.c_int, i32p, i32p, ctypes.c_uint32,
                               ctypes.POINTER(ctypes.c_int16), ctypes.c_uint32]

    def run(which, xs, table=None):
        xs = np.ascontiguousarray(xs, np.int32)
        out = np.zeros_like(xs)
        tp = None
        tl = 0
        if table is not None:
            table = np.ascontiguousarray(table, np.int16)
            tp = table.ctypes.data_as(ctypes.POINTER(ctypes.c_int16))
            tl = table.size
        rc = lib.prims_eval(which, xs.ctypes.data_as(i32p), out.ctypes.data_as(i32p),
                            xs.size, tp, tl)
        assert rc == 0, rc
        return out
    return run


@pytest.fixture(autouse=True)
def _reference_tables():
    orc.set_exp_policy(orc.EXP_HLS, orc.EXP_HLS)
    yield


def _oracle(fn, xs):
    return np.array([fn(int(x)) for x in xs], np.int32)


ALL16 = np.arange(-32768, 32768, dtype=np.int32)


def _int32_sweep(thresholds):
    """Every value below 2^16, one pseudo-random value in each 2^16-wide
    band of int32, and each threshold with its neighbours."""
    low = np.arange(0, 65536, dtype=np.int64)
    hi = np.arange(-32768, 32768, dtype=np.int64) << 16
    bands = hi + ((np.arange(65536, dtype=np.int64) * 2654435761) & 0xffff)
    th = np.array([t + d for t in thresholds for d in (-1, 0, 1)], np.int64)
    ext = np.array([-(1 << 31), (1 << 31) - 1, -1, 0, 1], np.int64)
    v = np.concatenate([low, bands, th, ext])
    v = v[(v >= -(1 << 31)) & (v < (1 << 31))]
    return np.unique(v).astype(np.int32)


def test_recip_every_int16(prims):
    got = prims(P_RECIP, ALL16)
    want = _oracle(orc.lib.orc_recip, ALL16)
    assert np.array_equal(got, want), np.flatnonzero(got != want)[:8]


def test_silu_every_int16(prims):
    import llm_accel
    e8, _ = llm_accel.exp_tables()
    got = prims(P_SILU, ALL16, e8)
    want = _oracle(orc.lib.orc_silu, ALL16)
    assert np.array_equal(got, want), np.flatnonzero(got != want)[:8]


def test_rsqrt_sweep(prims):
    xs = _int32_sweep([16, 4096, 16384, 1 << 16, 4 << 16, 16 << 16, 64 << 16])
    got = prims(P_RSQRT, xs)
    want = _oracle(orc.lib.orc_rsqrt, xs)
    assert np.array_equal(got, want), xs[np.flatnonzero(got != want)[:8]]


def test_inv_sum_sweep(prims):
    xs = _int32_sweep([16, 511, 512, 513, 1 << 16, 1 << 24])
    got = prims(P_INV_SUM, xs)
    want = _oracle(orc.lib.orc_inv_sum, xs)
    assert np.array_equal(got, want), xs[np.flatnonzero(got != want)[:8]]


def test_product_term_saturation_correction(prims):
    """a * golden_weight_t(b) narrowed to Q16.16: every int16 a against b
    at and around the Q4.12 saturation bounds, and every int16 b against
    extreme and swept a."""
    bs = np.array([-32768, -2049, -2048, -2047, -1, 0, 1, 2047, 2048, 2049, 4096,
                   32767], np.int32)
    as_ = np.array([-32768, -32767, -9, -8, -7, -1, 0, 1, 7, 8, 9, 23, 24, 25,
                    32766, 32767], np.int32)
    a1 = np.repeat(ALL16, bs.size)
    b1 = np.tile(bs, ALL16.size)
    b2 = np.repeat(ALL16, as_.size)
    a2 = np.tile(as_, ALL16.size)
    a = np.concatenate([a1, a2])
    b = np.concatenate([b1, b2])
    packed = ((a & 0xffff) | ((b & 0xffff) << 16)).astype(np.uint32).view(np.int32)
    got = prims(P_TERM, packed)
    want = np.array([orc.lib.orc_fm_wt_term(int(x), int(y)) for x, y in zip(a, b)],
                    np.int32)
    bad = np.flatnonzero(got != want)
    assert bad.size == 0, [(int(a[i]), int(b[i]), int(got[i]), int(want[i])) for i in bad[:8]]


def test_probability_every_difference(prims):
    import llm_accel
    _, e14 = llm_accel.exp_tables()
    xs = np.arange(-70000, 1, dtype=np.int32)
    got = prims(P_PROB, xs, e14)
    want = _oracle(lambda x: orc.lib.orc_attn_prob(max(-32768, x)), xs)
    assert np.array_equal(got, want), xs[np.flatnonzero(got != want)[:8]]
