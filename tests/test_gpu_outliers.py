"""Weights of any magnitude: the exact-sum paths of the VALU projections.

The reference accumulates every projection in 48 bits whatever the weights
(kernel/mm_stream_8x64_fused_mac.cpp:89-96).  The VALU kernels here keep
int32 partial sums over an interval of k-steps chosen from the matrix's
largest |weight| (8 products per lane per step, any int16 activation):
max|w| < 2048 raw (0.5) widens after 4 or more steps, [2048, 8192) after
every step, and from 8192 raw (2.0) up every product is widened.  A real
checkpoint with one outlier takes the slower intervals, so this runs a P8
block, two decode forwards and the LM head of a Qwen2.5-3B-shaped layer
whose every matrix holds such weights, against the oracle, and checks that
decode rows still take the fused attention sublayer -- on the 16-bit
layout (LLM_ACCEL_P12=0: the widening intervals) and on the 12-bit images,
where these few weights per row stay in the image clamped and their rows'
sparse corrections add the difference.
"""
import sys

import numpy as np
import pytest

from oracle import orc
import workloads
from helpers import accel_shape, first_mismatch, oracle_from_synthetic, oracle_shape

pytestmark = pytest.mark.gpu


def _say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def _plant(w, rng, value):
    """A few entries of magnitude `value` (both signs): the first and last
    element and random positions."""
    n, k = w.shape
    w[0, 0] = value
    w[n - 1, k - 1] = -value
    for _ in range(6):
        w[rng.integers(0, n), rng.integers(0, k)] = value if rng.integers(0, 2) else -value


@pytest.mark.parametrize("layout", ["16-bit", "12-bit"])
@pytest.mark.parametrize("value,interval", [(32767, "per product"), (4095, "per step"),
                                            (1500, "four steps")])
def test_outlier_weights_p8_decode_lm_head(value, interval, layout, monkeypatch):
    import llm_accel
    if layout == "16-bit":
        monkeypatch.setenv("LLM_ACCEL_P12", "0")
    spec = workloads.CONFIG_B
    max_seq = 64
    synth = workloads.SyntheticModel(spec, layers=1)
    rng = np.random.default_rng(value)
    for p in range(7):
        _plant(synth.weight(0, p), rng, value)
    om = oracle_from_synthetic(synth, oracle_shape(spec, layers=1, max_seq=max_seq))
    kv = om.new_kv()
    head = synth.lm_head()[:8192].copy()
    _plant(head, rng, value)
    hidden = synth.hidden_rows(10)
    with llm_accel.Accelerator(accel_shape(spec, layers=1, max_seq=max_seq)) as acc:
        acc.load_model(synth)
        acc.load_lm_head(head)
        if layout == "12-bit" and value > 2047:  # every matrix stays in 12 bits
            assert acc.weight_bytes()[1] == 0
        for pos, rows in ((0, 8), (8, 1), (9, 1)):
            _say(f"case outliers {value} ({interval}) {layout} pos={pos} rows={rows}")
            cur = hidden[pos:pos + rows]
            acc.upload(1, cur)
            acc.kernel_timing(True)
            for op, pin, pout in ((18, 1, 0), (19, 0, 1), (20, 1, 0)):
                code, want, _ = om.task(kv, op, 0, cur, pos)
                assert code == 0
                rc, _ = acc.task(op, 0, rows, pos, pin, pout)
                assert rc == 0
                err = first_mismatch(acc.download(pout, rows), want)
                assert err is None, f"op {op}: {err}"
                cur = want
            stats = acc.kernel_stats()
            acc.kernel_timing(False)
            if rows == 1:  # one launch for the decode row, not the separate kernels
                assert stats["attn_sublayer"][0] >= 1, stats
                assert stats["attention"][0] == 0 and stats["qkv"][0] == 0, stats
            toks, scores = acc.lm_head_argmax(0, 0, rows)
            assert toks == [orc.lm_head_argmax(head, cur[r]) for r in range(rows)]
        for h in range(spec.kv_heads):
            gk, gv = acc.kv_read(0, h, 0, 10)
            assert np.array_equal(gk, kv[0][0, h, :10])
            assert np.array_equal(gv, kv[1][0, h, :10])
