"""The chunked attention pair (attention_scores_kernel, attention_pv_kernel):
head_dim not a multiple of 32 with more tiles than one chunk (4 tiles).
Shapes with head_dim 48 and 16 over a 10-tile cache preloaded with seeded
K/V; 8-row blocks, pairs and single rows at positions that cross tile and
chunk boundaries, each task against the oracle, then the whole cache."""
import sys

import numpy as np
import pytest

import workloads
from helpers import accel_shape, first_mismatch, oracle_from_synthetic, oracle_shape

pytestmark = pytest.mark.gpu

MAX_SEQ = 640  # 10 tiles: 3 chunks of up to 4


def _say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


SPECS = {
    48: workloads.ShapeSpec("d48", 512, 192, 512, 1, 4, 2, MAX_SEQ, w_range=0.25,
                            emb_sigma=0.5),
    16: workloads.ShapeSpec("d16", 512, 128, 256, 1, 8, 2, MAX_SEQ, w_range=0.25,
                            emb_sigma=0.5),
}


@pytest.mark.parametrize("head_dim", [48, 16])
def test_chunked_attention_matches_oracle(head_dim):
    import llm_accel
    spec = SPECS[head_dim]
    assert spec.head_dim == head_dim
    synth = workloads.SyntheticModel(spec, layers=1)
    om = oracle_from_synthetic(synth, oracle_shape(spec, layers=1, max_seq=MAX_SEQ))
    kv = om.new_kv()
    pre = [synth.kv_rows(MAX_SEQ, seed_offset=40 + h) for h in range(spec.kv_heads)]
    schedule = [(252, 8), (300, 2), (383, 1), (384, 8), (511, 2), (513, 1), (600, 8),
                (631, 1)]
    hidden = synth.hidden_rows(sum(r for _, r in schedule))
    with llm_accel.Accelerator(accel_shape(spec, layers=1, max_seq=MAX_SEQ)) as acc:
        acc.load_model(synth)
        for h, (k, v) in enumerate(pre):
            acc.kv_write(0, h, 0, k, v)
            kv[0][0, h, :] = k
            kv[1][0, h, :] = v
        row0 = 0
        for pos, rows in schedule:
            h = hidden[row0:row0 + rows]
            row0 += rows
            _say(f"case chunked d={head_dim} pos={pos} rows={rows}")
            acc.upload(2, h)
            acc.kernel_timing(True)
            cur = h
            for op, pin, pout in ((18, 2, 0), (19, 0, 1), (20, 1, 0)):
                code, want, _ = om.task(kv, op, 0, cur, pos)
                assert code == 0
                rc, _ = acc.task(op, 0, rows, pos, pin, pout)
                assert rc == 0
                err = first_mismatch(acc.download(pout, rows), want)
                assert err is None, f"d={head_dim} pos {pos} rows {rows} op {op}: {err}"
                cur = want
            stats = acc.kernel_stats()
            acc.kernel_timing(False)
            # one attention launch (the scores / PV pair: every position
            # here lies beyond one chunk), not the fused sublayer
            assert stats["attention"][0] == 1 and stats["attn_sublayer"][0] == 0, stats
        for hh in range(spec.kv_heads):
            k, v = acc.kv_read(0, hh, 0, MAX_SEQ)
            assert first_mismatch(k, kv[0][0, hh]) is None, f"K head {hh}"
            assert first_mismatch(v, kv[1][0, hh]) is None, f"V head {hh}"
