"""llm_lm_head_argmax_static, the LM-head argmax that allocates nothing,
against the context entry point llm_lm_head_argmax on the same table and
rows: two calls in a row, the second smaller, both bit-exact."""
import ctypes

import numpy as np
import pytest

import llm_accel
import workloads
from helpers import accel_shape


class _Hip:
    """Device buffers through the HIP runtime the library itself links
    (libamdhip64.so.7): a second runtime in the process, such as torch's
    bundled one, cannot initialise once this one has."""

    def __init__(self):
        self.rt = ctypes.CDLL("libamdhip64.so.7")
        self.bufs = []
        assert self.rt.hipSetDevice(0) == 0

    def alloc(self, nbytes):
        p = ctypes.c_void_p()
        assert self.rt.hipMalloc(ctypes.byref(p), ctypes.c_size_t(nbytes)) == 0
        self.bufs.append(p)
        return p

    def to_device(self, a):
        a = np.ascontiguousarray(a)
        p = self.alloc(a.nbytes)
        assert self.rt.hipMemcpy(p, a.ctypes.data_as(ctypes.c_void_p),
                                 ctypes.c_size_t(a.nbytes), 1) == 0
        return p

    def to_host(self, p, like):
        assert self.rt.hipMemcpy(like.ctypes.data_as(ctypes.c_void_p), p,
                                 ctypes.c_size_t(like.nbytes), 2) == 0
        return like

    def sync(self):
        assert self.rt.hipDeviceSynchronize() == 0

    def free(self):
        for p in self.bufs:
            self.rt.hipFree(p)
        self.bufs = []


def _call(hip, table_dev, vocab, hidden, rows_dev, ld, nrows):
    tok = hip.to_device(np.full(8, -1, np.int32))
    sc = hip.to_device(np.zeros(8, np.int64))
    rc = llm_accel.lib().llm_lm_head_argmax_static(
        table_dev, vocab, hidden, rows_dev, ld, nrows, tok, sc, None)
    assert rc == 0, llm_accel.lib().llm_last_error()
    hip.sync()
    toks = hip.to_host(tok, np.zeros(8, np.int32))
    scores = hip.to_host(sc, np.zeros(8, np.int64))
    assert (toks[nrows:] == -1).all()  # rows beyond row_count untouched
    return toks[:nrows].astype(np.uint32).tolist(), scores[:nrows].tolist()


def _table_and_rows(rng, vocab, hidden):
    table = rng.integers(-600, 601, (vocab, hidden)).astype(np.int16)
    rows = rng.integers(-3000, 3001, (8, hidden)).astype(np.int16)
    # row 0 saturates: the extreme product (-32768) * (-32767) on every
    # column, won by two identical table rows (first index must win)
    rows[0] = -32768
    table[70] = -32767
    table[vocab - 5] = -32767
    # row 1: two equal maxima far apart
    table[11] = np.where(rows[1] >= 0, 900, -900)
    table[vocab - 2] = table[11]
    return table, rows


@pytest.mark.gpu
def test_static_argmax_matches_context_argmax_twice():
    rng = np.random.default_rng(20260718)
    spec = workloads.CONFIG_A
    H = spec.hidden
    V1, V2 = 5000, 1800
    table, rows = _table_and_rows(rng, V1, H)
    with llm_accel.Accelerator(accel_shape(spec, layers=1, max_seq=64)) as acc:
        hip = _Hip()
        try:
            table_dev = hip.to_device(table)
            rows_dev = hip.to_device(rows)
            acc.load_lm_head(table)
            acc.upload(0, rows)
            ref = acc.lm_head_argmax(0, 0, 8)
            got = _call(hip, table_dev, V1, H, rows_dev, H, 8)
            assert got == ref
            assert ref[0][0] == 70 and ref[0][1] == 11

            # second call: a smaller vocabulary (a prefix of the table),
            # three rows with a row stride wider than hidden
            rows2 = rng.integers(-3000, 3001, (3, H)).astype(np.int16)
            ld = H + 8
            padded = np.zeros((3, ld), np.int16)
            padded[:, :H] = rows2
            rows2_dev = hip.to_device(padded)
            acc.load_lm_head(table[:V2])
            acc.upload(1, rows2)
            ref2 = acc.lm_head_argmax(1, 0, 3)
            got2 = _call(hip, table_dev, V2, H, rows2_dev, ld, 3)
            assert got2 == ref2
        finally:
            hip.free()


def test_static_argmax_rejects_sizes_beyond_its_limits():
    lib = llm_accel.lib()
    p = ctypes.c_void_p(1 << 20)  # aligned, never dereferenced: rejected first
    cases = [
        (5000, 256, 256, 9),       # more rows than the scratch holds
        (5000, 16392, 16392, 1),   # hidden beyond 16384
        (1 << 18, 256, 256, 1),    # vocab beyond the key's index field
        (5000, 250, 256, 1),       # hidden not a multiple of 8
        (5000, 256, 252, 1),       # ld < hidden
        (5000, 256, 256, 0),       # no rows
    ]
    for vocab, hidden, ld, nrows in cases:
        rc = lib.llm_lm_head_argmax_static(p, vocab, hidden, p, ld, nrows, p, None,
                                           None)
        assert rc == -1, (vocab, hidden, ld, nrows)  # LLM_E_ARG
        assert lib.llm_last_error()
