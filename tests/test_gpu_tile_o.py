"""Decode rows at 5-64 tiles: the one-launch tile path and the O projection
in one launch (tile workgroups, then O blocks waiting for every query
head's attention row).  Task 18 must equal the oracle bit for bit with the
launch on and off (LLM_ACCEL_TILE_O), on the 12-bit weights and with O (and
Q|K|V, read with it) widened to 16 bits by one out-of-range weight, and the
K/V rows it appends must be the oracle's."""
import os
import sys

import numpy as np
import pytest

import workloads
from helpers import accel_shape, first_mismatch, oracle_from_synthetic, oracle_shape
from test_gpu_p12 import _Edited, _extremes, _outlier

pytestmark = pytest.mark.gpu


def _say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def _accel(spec, env, max_seq):
    import llm_accel
    old = {k: os.environ.get(k) for k in env}
    os.environ.update(env)
    try:
        return llm_accel.Accelerator(accel_shape(spec, layers=1, max_seq=max_seq))
    finally:
        for k, v in old.items():
            if v is None:
                os.environ.pop(k, None)
            else:
                os.environ[k] = v


@pytest.mark.parametrize("cfg", ["A", "B"])
@pytest.mark.parametrize("case", ["extremes", "o_outlier"])
def test_tile_o_matches_oracle(cfg, case):
    spec = workloads.CONFIG_A if cfg == "A" else workloads.CONFIG_B
    lengths = (300, 1100, 1400)  # 6, 18 and 22 tiles: the grid fits at 1-2 rows
    nmax = max(lengths) + 8
    synth = workloads.SyntheticModel(spec, layers=1)
    edits = {(0, p): _extremes for p in range(4)}
    if case == "o_outlier":
        edits[(0, 3)] = _outlier
    model = _Edited(synth, edits)
    om = oracle_from_synthetic(model, oracle_shape(spec, layers=1, max_seq=nmax))
    pre = [synth.kv_rows(nmax, seed_offset=40 + h) for h in range(spec.kv_heads)]
    rng = np.random.default_rng(18)
    cases = [(n, rows, rng.integers(-20000, 20000, (rows, spec.hidden)).astype(np.int16))
             for n in lengths for rows in (1, 2)]
    want = {}
    for n, rows, x in cases:
        kc, vc = om.new_kv()
        for h in range(spec.kv_heads):
            kc[0, h, :n], vc[0, h, :n] = pre[h][0][:n], pre[h][1][:n]
        code, out, _ = om.task((kc, vc), 18, 0, x, n)
        assert code == 0
        want[(n, rows)] = (out, [(kc[0, h, n:n + rows].copy(), vc[0, h, n:n + rows].copy())
                                 for h in range(spec.kv_heads)])
    for tile_o in ("1", "0"):
        with _accel(spec, {"LLM_ACCEL_TILE_O": tile_o}, nmax) as acc:
            acc.load_model(model)
            for n, rows, x in cases:
                for h in range(spec.kv_heads):
                    acc.kv_write(0, h, 0, pre[h][0][:n], pre[h][1][:n])
                acc.upload(2, x)
                _say(f"case tile_o={tile_o} {cfg} {case} n={n} rows={rows}")
                acc.kernel_timing(True)
                rc, _ = acc.task(18, 0, rows, n, 2, 0)
                assert rc == 0
                stats = acc.kernel_stats()
                acc.kernel_timing(False)
                # one launch for attention and O when on, two when off
                assert stats["attention"][0] == 1, stats
                assert stats["oproj"][0] == (0 if tile_o == "1" else 1), stats
                got = acc.download(0, rows)
                out, kv = want[(n, rows)]
                assert first_mismatch(got, out) is None, f"tile_o={tile_o} n={n} rows={rows}"
                for h in range(spec.kv_heads):
                    k, v = acc.kv_read(0, h, n, rows)
                    assert np.array_equal(k, kv[h][0]) and np.array_equal(v, kv[h][1])
