"""12-bit weight copies of the FFN matrices (single decode rows; 2-row
blocks keep the 16-bit kernel and are checked here too):
every weight w in [-2048, 2047] is read as w + 2048 = 256 h + l, the sums
are exact integers, so Task 19 must equal the oracle (and the 16-bit path)
bit for bit; a matrix with any weight outside that range keeps the 16-bit
copy."""
import os
import sys

import numpy as np
import pytest

import workloads
from helpers import accel_shape, first_mismatch, oracle_from_synthetic, oracle_shape

pytestmark = pytest.mark.gpu


def _say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


class _Edited:
    """A SyntheticModel with some FFN weights replaced."""

    def __init__(self, synth, edits):
        self._s = synth
        self._w = {}
        for (layer, proj), fn in edits.items():
            w = synth.weight(layer, proj).copy()
            fn(w)
            self._w[(layer, proj)] = w

    def weight(self, layer, proj):
        return self._w.get((layer, proj), self._s.weight(layer, proj))

    def norms(self):
        return self._s.norms()


def _accel(spec, env):
    import llm_accel
    old = {k: os.environ.get(k) for k in env}
    os.environ.update(env)
    try:
        return llm_accel.Accelerator(accel_shape(spec, layers=1, max_seq=64))
    finally:
        for k, v in old.items():
            if v is None:
                os.environ.pop(k, None)
            else:
                os.environ[k] = v


def _extremes(w):
    flat = w.reshape(-1)
    flat[::97] = -2048
    flat[13::89] = 2047


def _outlier(w):
    _extremes(w)
    w[w.shape[0] // 2, 5] = 2048  # one weight past 12 bits


@pytest.mark.parametrize("cfg", ["A", "B"])
@pytest.mark.parametrize("case", ["extremes", "down_outlier", "gate_outlier"])
def test_ffn_p12_matches_oracle_and_16bit(cfg, case):
    spec = workloads.CONFIG_A if cfg == "A" else workloads.CONFIG_B
    synth = workloads.SyntheticModel(spec, layers=1)
    edits = {(0, 4): _extremes, (0, 5): _extremes, (0, 6): _extremes}
    if case == "down_outlier":
        edits[(0, 6)] = _outlier
    if case == "gate_outlier":
        edits[(0, 4)] = _outlier
    model = _Edited(synth, edits)
    om = oracle_from_synthetic(model, oracle_shape(spec, layers=1, max_seq=64))
    rng = np.random.default_rng(5)
    outs = {}
    for p12 in ("1", "0"):
        with _accel(spec, {"LLM_ACCEL_P12": p12}) as acc:
            acc.load_model(model)
            got = []
            for rows in (1, 2):
                h = rng.integers(-32768, 32768, (rows, spec.hidden)).astype(np.int16) \
                    if p12 == "1" else outs[("h", rows)]
                outs[("h", rows)] = h
                acc.upload(2, h)
                _say(f"case {cfg} {case} p12={p12} rows={rows}")
                rc, _ = acc.task(19, 0, rows, 0, 2, 0)
                assert rc == 0
                got.append(acc.download(0, rows))
            outs[p12] = got
    for k, rows in enumerate((1, 2)):
        kv = om.new_kv()
        code, want, _ = om.task(kv, 19, 0, outs[("h", rows)], 0)
        assert code == 0
        assert first_mismatch(outs["1"][k], want) is None, f"p12 rows={rows}"
        assert first_mismatch(outs["0"][k], want) is None, f"16-bit rows={rows}"


@pytest.mark.parametrize("n", [300, 100])
@pytest.mark.parametrize("cfg", ["A", "B"])
@pytest.mark.parametrize("case", ["extremes", "v_outlier", "o_outlier"])
def test_attention_p12_matches_oracle_and_16bit(cfg, case, n):
    """Task 18 of one row over Q / K / V / O weights that reach -2048 and
    2047; one weight past 12 bits in V (the whole Q|K|V matrix keeps 16
    bits) or in O.  At 300 positions (5 tiles) QKV, attention and O are
    separate launches on the 12-bit copies (the QKV launch normalises its
    input on load); at 100 (2 tiles) they are the fused sublayer's roles,
    which keep the 16-bit layout (their chain is bound by round trips, not
    bytes)."""
    spec = workloads.CONFIG_A if cfg == "A" else workloads.CONFIG_B
    synth = workloads.SyntheticModel(spec, layers=1)
    edits = {(0, p): _extremes for p in range(4)}
    if case == "v_outlier":
        edits[(0, 2)] = _outlier
    if case == "o_outlier":
        edits[(0, 3)] = _outlier
    model = _Edited(synth, edits)
    om = oracle_from_synthetic(model, oracle_shape(spec, layers=1, max_seq=n + 8))
    kc, vc = om.new_kv()
    pre = [synth.kv_rows(n, seed_offset=90 + h) for h in range(spec.kv_heads)]
    for h in range(spec.kv_heads):
        kc[0, h, :n], vc[0, h, :n] = pre[h]
    x = np.random.default_rng(6).integers(-20000, 20000, (1, spec.hidden)).astype(np.int16)
    outs = {}
    for p12 in ("1", "0"):
        import llm_accel
        old = {k: os.environ.get(k) for k in ("LLM_ACCEL_P12",)}
        os.environ.update({"LLM_ACCEL_P12": p12})
        try:
            acc = llm_accel.Accelerator(accel_shape(spec, layers=1, max_seq=n + 8))
        finally:
            for k, v in old.items():
                if v is None:
                    os.environ.pop(k, None)
                else:
                    os.environ[k] = v
        with acc:
            acc.load_model(model)
            for h in range(spec.kv_heads):
                acc.kv_write(0, h, 0, *pre[h])
            acc.upload(2, x)
            _say(f"case attention {cfg} {case} n={n} p12={p12}")
            acc.kernel_timing(True)
            rc, _ = acc.task(18, 0, 1, n, 2, 0)
            assert rc == 0
            outs[p12] = (acc.download(0, 1), [acc.kv_read(0, h, n, 1)
                                              for h in range(spec.kv_heads)])
            stats = acc.kernel_stats()
            acc.kernel_timing(False)
            assert stats["attn_sublayer"][0] == (1 if n <= 192 else 0), stats
    code, want, _ = om.task((kc, vc), 18, 0, x, n)
    assert code == 0
    for p12 in ("1", "0"):
        got, kv = outs[p12]
        assert first_mismatch(got, want) is None, f"p12={p12}"
        for h in range(spec.kv_heads):
            assert np.array_equal(kv[h][0], kc[0, h, n:n + 1])
            assert np.array_equal(kv[h][1], vc[0, h, n:n + 1])
