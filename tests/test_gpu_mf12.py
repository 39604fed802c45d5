"""Matrix-core projections of blocks of 3+ rows over the 12-bit weight
copies (LLM_ACCEL_MF12=1, the default) and over the byte planes
(LLM_ACCEL_MF12=0): both give the exact int64 sums, so Tasks 18 and 19 must
equal the oracle bit for bit either way.  Weights reach -2048 and 2047; a
matrix with a weight past 12 bits has no 12-bit copy and keeps the byte
planes in both runs.  Config A's down projection has K = 688 (11 K chunks
of 64 in 6 k-steps of 128: the last step's second half carries no
weights)."""
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
@pytest.mark.parametrize("case", ["extremes", "gate_outlier"])
def test_ffn_mf12_matches_oracle(cfg, case):
    spec = workloads.CONFIG_A if cfg == "A" else workloads.CONFIG_B
    synth = workloads.SyntheticModel(spec, layers=1)
    edits = {(0, 4): _extremes, (0, 5): _extremes, (0, 6): _extremes}
    if case == "gate_outlier":
        edits[(0, 4)] = _outlier
    model = _Edited(synth, edits)
    om = oracle_from_synthetic(model, oracle_shape(spec, layers=1, max_seq=64))
    rng = np.random.default_rng(15)
    hs = {rows: rng.integers(-32768, 32768, (rows, spec.hidden)).astype(np.int16)
          for rows in (3, 5, 8)}
    for mf12 in ("1", "0"):
        with _accel(spec, {"LLM_ACCEL_MF12": mf12}, 64) as acc:
            acc.load_model(model)
            for rows, h in hs.items():
                acc.upload(2, h)
                _say(f"case ffn {cfg} {case} mf12={mf12} rows={rows}")
                rc, _ = acc.task(19, 0, rows, 0, 2, 0)
                assert rc == 0
                got = acc.download(0, rows)
                code, want, _ = om.task(om.new_kv(), 19, 0, h, 0)
                assert code == 0
                assert first_mismatch(got, want) is None, f"mf12={mf12} rows={rows}"


@pytest.mark.parametrize("cfg", ["A", "B"])
@pytest.mark.parametrize("case", ["extremes", "o_outlier"])
def test_attention_mf12_matches_oracle(cfg, case):
    """Task 18 of 3 and 8 rows after 300 cached positions: the Q|K|V
    projection (normalising its input on load where the gain is constant)
    and O on the matrix cores."""
    n = 300
    spec = workloads.CONFIG_A if cfg == "A" else workloads.CONFIG_B
    synth = workloads.SyntheticModel(spec, layers=1)
    edits = {(0, p): _extremes for p in range(4)}
    if case == "o_outlier":
        edits[(0, 3)] = _outlier
    model = _Edited(synth, edits)
    om = oracle_from_synthetic(model, oracle_shape(spec, layers=1, max_seq=n + 16))
    pre = [synth.kv_rows(n, seed_offset=70 + h) for h in range(spec.kv_heads)]
    rng = np.random.default_rng(16)
    xs = {rows: rng.integers(-20000, 20000, (rows, spec.hidden)).astype(np.int16)
          for rows in (3, 8)}
    want = {}
    for rows, x in xs.items():
        kc, vc = om.new_kv()
        for h in range(spec.kv_heads):
            kc[0, h, :n], vc[0, h, :n] = pre[h]
        code, out, _ = om.task((kc, vc), 18, 0, x, n)
        assert code == 0
        want[rows] = out
    for mf12 in ("1", "0"):
        with _accel(spec, {"LLM_ACCEL_MF12": mf12}, n + 16) as acc:
            acc.load_model(model)
            for rows, x in xs.items():
                for h in range(spec.kv_heads):
                    acc.kv_write(0, h, 0, *pre[h])
                acc.upload(2, x)
                _say(f"case attention {cfg} {case} mf12={mf12} rows={rows}")
                rc, _ = acc.task(18, 0, rows, n, 2, 0)
                assert rc == 0
                got = acc.download(0, rows)
                assert first_mismatch(got, want[rows]) is None, f"mf12={mf12} rows={rows}"


def _dense(w):
    """Five weights past 12 bits in one row: more than a row's corrections
    hold."""
    _extremes(w)
    w[w.shape[0] // 3, 1:6] = 3000


# case: (edits, matrices held in 16 bits, matrices with corrections)
_IMAGE_CASES = {
    "fits": ({}, [], []),
    "down_outlier": ({6: _outlier}, [], ["down"]),
    "v_outlier": ({2: _outlier}, [], ["qkv"]),
    "gate_outlier": ({4: _outlier}, [], ["gate"]),
    "dense_down": ({6: _dense}, ["down"], []),
    "dense_v_after_q_outlier": ({0: _outlier, 2: _dense}, ["qkv", "o"], []),
    "dense_up": ({5: _dense}, ["gate", "up"], []),
}


@pytest.mark.parametrize("case", list(_IMAGE_CASES))
def test_single_weight_image(case):
    """Matrices whose weights fit 12 bits hold only the 12-bit copy and the
    byte sums.  Rows with at most 4 weights past 12 bits keep the image:
    the copy holds the weights clamped and the row's correction words the
    differences, which every 12-bit kernel adds exactly.  More in a row
    moves the matrix and the one read with it (gate with up, Q|K|V with O)
    to the 16-bit tiles and byte planes, rebuilt from what was loaded --
    corrections included (V arrives after Q and K of the same Q|K|V
    matrix).  Task 18 + 19 of 1, 2 and 8 rows must still equal the
    oracle."""
    spec = workloads.CONFIG_A
    synth = workloads.SyntheticModel(spec, layers=1)
    edits_p, wide_names, corr_names = _IMAGE_CASES[case]
    edits = {(0, p): _extremes for p in range(7)}
    for p, fn in edits_p.items():
        edits[(0, p)] = fn
    model = _Edited(synth, edits)
    om = oracle_from_synthetic(model, oracle_shape(spec, layers=1, max_seq=64))
    kpad = {"qkv": 256, "o": 256, "gate": 256, "up": 256, "down": 768}
    npad = {"qkv": 512, "o": 256, "gate": 688, "up": 688, "down": 256}
    kq = {"qkv": 4, "o": 4, "gate": 4, "up": 4, "down": 11}
    rng = np.random.default_rng(17)
    with _accel(spec, {}, 64) as acc:
        acc.load_model(model)
        nbytes, wide = acc.weight_bytes()
        want_bytes = 0
        for name in npad:
            elems = npad[name] * kpad[name]
            nc = -(-npad[name] // 16)
            want_bytes += nc * 16 * 2 * 4
            if name in wide_names:
                want_bytes += elems * 2 + nc * kq[name] * 2048
            else:
                want_bytes += elems // 512 * 768
            if name in corr_names:
                want_bytes += npad[name] * 4 * 4
        _say(f"case single image {case}: {nbytes} bytes, {wide} wide")
        assert wide == len(wide_names)
        assert nbytes == want_bytes
        for rows in (1, 2, 8):
            h = rng.integers(-20000, 20000, (rows, spec.hidden)).astype(np.int16)
            kc, vc = om.new_kv()
            acc.kv_clear()
            acc.upload(2, h)
            rc, _ = acc.task(18, 0, rows, 0, 2, 0)
            assert rc == 0
            rc, _ = acc.task(19, 0, rows, 0, 0, 1)
            assert rc == 0
            got = acc.download(1, rows)
            code, mid, _ = om.task((kc, vc), 18, 0, h, 0)
            assert code == 0
            code, want, _ = om.task((kc, vc), 19, 0, mid, 0)
            assert code == 0
            assert first_mismatch(got, want) is None, f"{case} rows={rows}"
