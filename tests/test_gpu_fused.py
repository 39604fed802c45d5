"""Fused attention sublayer: QKV projection, attention and O projection of
decode rows in one launch (the reference runs them as steps 0-3 of one
Task 18, kernel/control_cache_8x64.cpp:5974-6164).  It engages where it
applies, agrees bit for bit with the separate launches and with the
oracle, and a wait between its workgroups that gives up is reported at the
next synchronisation and leaves the context usable."""
import os
import sys

import pytest

import workloads
from helpers import accel_shape, first_mismatch, oracle_from_synthetic, oracle_shape

pytestmark = pytest.mark.gpu


def _say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def _accel(spec, layers, max_seq, env):
    """A context created with `env` set (read once, at creation)."""
    import llm_accel
    env = dict(env)
    old = {k: os.environ.get(k) for k in env}
    os.environ.update(env)
    try:
        return llm_accel.Accelerator(accel_shape(spec, layers=layers, max_seq=max_seq))
    finally:
        for k, v in old.items():
            if v is None:
                os.environ.pop(k, None)
            else:
                os.environ[k] = v


def _forward(acc, layers, rows, pos, pair_in=2):
    """T18 / T19 over every layer; returns the hidden rows after each task."""
    outs = []
    pin, pout = pair_in, 0
    for layer in range(layers):
        for op in (18, 19):
            rc, _ = acc.task(op, layer, rows, pos, pin, pout)
            assert rc == 0
            outs.append(acc.download(pout, rows))
            pin, pout = pout, pin
    return outs


def test_fused_sublayer_engages_for_decode_rows():
    """Decode rows (1 and 2) take the fused launch, an 8-row block does not;
    every task's rows equal the oracle's."""
    spec = workloads.CONFIG_B
    synth = workloads.SyntheticModel(spec, seed=workloads.SEED, layers=1)
    om = oracle_from_synthetic(synth, oracle_shape(spec, layers=1, max_seq=64))
    kv = om.new_kv()
    hidden = synth.hidden_rows(11)
    acc = _accel(spec, 1, 64, {"LLM_ACCEL_FUSED": "1"})
    with acc:
        acc.load_model(synth)
        for pos, rows in ((0, 8), (8, 1), (9, 2)):
            _say(f"case B pos={pos} rows={rows}")
            h = hidden[pos:pos + rows]
            acc.upload(2, h)
            acc.kernel_timing(True)
            rc, _ = acc.task(18, 0, rows, pos, 2, 0)
            assert rc == 0
            got = acc.download(0, rows)
            stats = acc.kernel_stats()
            acc.kernel_timing(False)
            code, want, _ = om.task(kv, 18, 0, h, pos)
            assert code == 0
            assert first_mismatch(got, want) is None
            fused = stats["attn_sublayer"][0]
            assert fused == (1 if rows <= 2 else 0), stats
            assert stats["attention"][0] == (0 if rows <= 2 else 1), stats
            rc, _ = acc.task(19, 0, rows, pos, 0, 1)
            code, want19, _ = om.task(kv, 19, 0, want, pos)
            assert first_mismatch(acc.download(1, rows), want19) is None


@pytest.mark.parametrize("cfg", ["A", "B"])
def test_fused_equals_separate_launches(cfg):
    """The same decode sequence through the fused launch and through the
    three separate launches: hidden rows after every task and the K/V cache
    agree bit for bit."""
    spec = workloads.CONFIG_A if cfg == "A" else workloads.CONFIG_B
    layers = 2
    synth = workloads.SyntheticModel(spec, seed=workloads.SEED + 7, layers=layers)
    schedule = [(0, 8), (8, 1), (9, 2), (11, 1), (12, 2)]
    hidden = synth.hidden_rows(14)
    results = []
    for fused in ("1", "0"):
        acc = _accel(spec, layers, 128, {"LLM_ACCEL_FUSED": fused})
        with acc:
            acc.load_model(synth)
            outs = []
            for pos, rows in schedule:
                _say(f"case {cfg} fused={fused} pos={pos} rows={rows}")
                acc.upload(2, hidden[pos:pos + rows])
                outs += _forward(acc, layers, rows, pos)
            kvs = [acc.kv_read(layer, h, 0, 14) for layer in range(layers)
                   for h in range(spec.kv_heads)]
            results.append((outs, kvs))
    (o1, k1), (o0, k0) = results
    for i, (a, b) in enumerate(zip(o1, o0)):
        assert first_mismatch(a, b) is None, f"task output {i}"
    for i, ((ka, va), (kb, vb)) in enumerate(zip(k1, k0)):
        assert first_mismatch(ka, kb) is None, f"K cache {i}"
        assert first_mismatch(va, vb) is None, f"V cache {i}"


def test_wait_time_out_is_reported_and_cleared():
    """With a wait bound of 0 ticks every wait of a fused launch gives up
    (the kernel still ends normally: every wait is bounded).  The next
    synchronisation reports it, the one after that is clean, and tasks that
    do not use the fused launch still match the oracle."""
    import llm_accel
    spec = workloads.CONFIG_B
    synth = workloads.SyntheticModel(spec, seed=workloads.SEED, layers=1)
    om = oracle_from_synthetic(synth, oracle_shape(spec, layers=1, max_seq=64))
    kv = om.new_kv()
    hidden = synth.hidden_rows(17)
    acc = _accel(spec, 1, 64, {"LLM_ACCEL_FUSED": "1", "LLM_ACCEL_WAIT_LIMIT": "0"})
    with acc:
        acc.load_model(synth)
        acc.upload(2, hidden[:8])
        _say("case B P8 block before the forced time-out")
        _forward(acc, 1, 8, 0)
        om.task(kv, 18, 0, hidden[:8], 0)
        acc.sync()
        acc.upload(3, hidden[8:9])
        _say("case B decode row with a 0-tick wait bound")
        rc, _ = acc.task(18, 0, 1, 8, 3, 0)
        assert rc == 0
        with pytest.raises(llm_accel.AccelError, match="timed out"):
            acc.sync()
        acc.sync()  # cleared
        # an 8-row block (separate launches) at a fresh position range
        _say("case B P8 block after the time-out")
        h = hidden[9:17]
        acc.upload(2, h)
        rc, _ = acc.task(18, 0, 8, 9, 2, 0)
        got = acc.download(0, 8)
        # the oracle's cache holds positions 0..7 and, like the aborted
        # launch's, no position 8 row: give it the GPU's row 8 (whatever
        # the aborted launch left) so that both attend over the same cache
        for hh in range(spec.kv_heads):
            k, v = acc.kv_read(0, hh, 8, 1)
            kv[0][0, hh, 8] = k[0]
            kv[1][0, hh, 8] = v[0]
        code, want, _ = om.task(kv, 18, 0, h, 9)
        assert code == 0
        assert first_mismatch(got, want) is None


@pytest.mark.parametrize("cfg", ["A", "B"])
def test_fused_rows_across_tile_boundaries(cfg):
    """Decode blocks of 1-2 rows in the fused launch at and across the
    boundaries of its 4 tiles (the block's own K/V rows split over two
    tiles, the last row of the 4th tile): every task's rows and every K/V
    row equal the oracle's."""
    spec = workloads.CONFIG_A if cfg == "A" else workloads.CONFIG_B
    schedule = [(63, 2), (127, 2), (128, 1), (191, 2), (254, 2)]
    synth = workloads.SyntheticModel(spec, seed=workloads.SEED + 13, layers=1)
    om = oracle_from_synthetic(synth, oracle_shape(spec, layers=1, max_seq=256))
    kv = om.new_kv()
    pre = [synth.kv_rows(256, seed_offset=70 + h) for h in range(spec.kv_heads)]
    hidden = synth.hidden_rows(2 * len(schedule))
    acc = _accel(spec, 1, 256, {"LLM_ACCEL_FUSED": "1"})
    with acc:
        acc.load_model(synth)
        for h, (k, v) in enumerate(pre):
            # every position the schedule does not write: preloaded
            acc.kv_write(0, h, 0, k, v)
            kv[0][0, h, :] = k
            kv[1][0, h, :] = v
        for i, (pos, rows) in enumerate(schedule):
            _say(f"case {cfg} fused rows={rows} at {pos}")
            h = hidden[2 * i:2 * i + rows]
            acc.upload(2, h)
            acc.kernel_timing(True)
            rc, _ = acc.task(18, 0, rows, pos, 2, 0)
            assert rc == 0
            got = acc.download(0, rows)
            assert acc.kernel_stats()["attn_sublayer"][0] == 1
            acc.kernel_timing(False)
            code, want, _ = om.task(kv, 18, 0, h, pos)
            assert code == 0
            assert first_mismatch(got, want) is None, f"rows {rows} at {pos}"
        for hh in range(spec.kv_heads):
            k, v = acc.kv_read(0, hh, 0, 256)
            assert first_mismatch(k, kv[0][0, hh]) is None, f"K head {hh}"
            assert first_mismatch(v, kv[1][0, hh]) is None, f"V head {hh}"


@pytest.mark.parametrize("start", [0, 0xFFFFFF80])
def test_fused_long_mixed_sequence(start):
    """A long sequence mixing fused launches (1-2 rows) with separate ones
    (8-row and 5-row blocks) over two layers, checked against the oracle
    after every task: the host's copies of the arrival counters stay in
    step with the device's.  Started just below 2^32 the counters wrap
    within a few launches (the waits compare modulo 2^32)."""
    spec = workloads.CONFIG_A
    layers = 2
    synth = workloads.SyntheticModel(spec, seed=workloads.SEED + 17, layers=layers)
    om = oracle_from_synthetic(synth, oracle_shape(spec, layers=layers, max_seq=128))
    kv = om.new_kv()
    schedule = [(0, 8)] + [(8 + i, 1) for i in range(6)] + [(14, 5)] + \
               [(19 + 2 * i, 2) for i in range(6)] + [(31, 1), (32, 8)] + \
               [(40 + i, 1) for i in range(6)]
    total = sum(r for _, r in schedule)
    hidden = synth.hidden_rows(total)
    acc = _accel(spec, layers, 128, {"LLM_ACCEL_FUSED": "1",
                                     "LLM_ACCEL_SYNC_START": str(start)})
    with acc:
        acc.load_model(synth)
        row0 = 0
        for pos, rows in schedule:
            h = hidden[row0:row0 + rows]
            row0 += rows
            _say(f"case A start={start:#x} pos={pos} rows={rows}")
            acc.upload(2, h)
            cur = h
            pin, pout = 2, 0
            for layer in range(layers):
                for op in (18, 19):
                    rc, _ = acc.task(op, layer, rows, pos, pin, pout)
                    assert rc == 0
                    code, want, _ = om.task(kv, op, layer, cur, pos)
                    assert code == 0
                    err = first_mismatch(acc.download(pout, rows), want)
                    assert err is None, f"op {op} layer {layer} at {pos}: {err}"
                    cur = want
                    pin, pout = pout, pin


@pytest.mark.parametrize("path", ["tile", "gqa"])
def test_tile_path_wait_timeout_is_reported(path):
    """The one-launch tile path, or the one-launch GQA path (scores and PV;
    forced from 5 tiles), for a decode row at 5 tiles with a 0-tick wait
    bound: the launch ends (every wait is bounded); either every wait was
    already satisfied at its first poll and the row equals the oracle's, or
    the next synchronisation reports the time-out and the one after is
    clean.  An 8-row block that does not wait (2 tiles) then matches the
    oracle."""
    import llm_accel
    spec = workloads.CONFIG_B
    n = 300
    synth = workloads.SyntheticModel(spec, seed=workloads.SEED, layers=1)
    om = oracle_from_synthetic(synth, oracle_shape(spec, layers=1, max_seq=512))
    kc, vc = om.new_kv()
    env = {"LLM_ACCEL_WAIT_LIMIT": "0"}
    if path == "gqa":
        env["LLM_ACCEL_GQA_MIN_TILES"] = "5"
    acc = _accel(spec, 1, 512, env)
    with acc:
        acc.load_model(synth)
        for h in range(spec.kv_heads):
            k, v = synth.kv_rows(n, seed_offset=80 + h)
            kc[0, h, :n], vc[0, h, :n] = k, v
            acc.kv_write(0, h, 0, k, v)
        x = synth.hidden_rows(1, seed_offset=81)
        acc.upload(2, x)
        _say(f"case {path} path 0-tick wait bound n={n}")
        rc, _ = acc.task(18, 0, 1, n, 2, 0)
        assert rc == 0
        try:
            acc.sync()
            timed_out = False
        except llm_accel.AccelError as e:
            assert "timed out" in str(e)
            timed_out = True
        acc.sync()  # clean either way
        if not timed_out:
            _, want, _ = om.task((kc, vc), 18, 0, x, n)
            assert first_mismatch(acc.download(0, 1), want) is None
        else:
            # the aborted launch may have appended position n on the GPU:
            # give the oracle the same row
            for h in range(spec.kv_heads):
                k, v = acc.kv_read(0, h, n, 1)
                kc[0, h, n], vc[0, h, n] = k[0], v[0]
        # an 8-row block at positions 100-107 (split-head path, no waits)
        h8 = synth.hidden_rows(8, seed_offset=82)
        acc.upload(3, h8)
        _say("case 8-row block after the tile-path wait")
        rc, _ = acc.task(18, 0, 8, 100, 3, 1)
        assert rc == 0
        got = acc.download(1, 8)
    kc2, vc2 = kc.copy(), vc.copy()
    code, want, _ = om.task((kc2, vc2), 18, 0, h8, 100)
    assert code == 0
    assert first_mismatch(got, want) is None


@pytest.mark.parametrize("path", ["tile", "gqa", "gqa_no_scan"])
def test_cooperative_launch_of_one_launch_kernels(path):
    """LLM_ACCEL_COOP=1: the one-launch tile and GQA kernels go through
    hipLaunchCooperativeKernel (a grid the device cannot hold at once is
    refused and the separate launches run instead).  Decode rows at 300 and
    700 positions and an 8-row block at 520 against the oracle, every
    appended K/V row included."""
    import llm_accel
    spec = workloads.CONFIG_B
    n = 700
    synth = workloads.SyntheticModel(spec, seed=workloads.SEED, layers=1)
    om = oracle_from_synthetic(synth, oracle_shape(spec, layers=1, max_seq=n + 16))
    kc, vc = om.new_kv()
    env = {"LLM_ACCEL_COOP": "1"}
    if path != "tile":
        env["LLM_ACCEL_GQA_MIN_TILES"] = "5"
    if path == "gqa_no_scan":
        env["LLM_ACCEL_GQA_SCAN_FUSED"] = "0"
    acc = _accel(spec, 1, n + 16, env)
    with acc:
        acc.load_model(synth)
        for h in range(spec.kv_heads):
            k, v = synth.kv_rows(n, seed_offset=90 + h)
            kc[0, h, :n], vc[0, h, :n] = k, v
            acc.kv_write(0, h, 0, k, v)
        for pos, rows in ((300, 1), (520, 8), (n, 1)):
            x = synth.hidden_rows(rows, seed_offset=91 + pos)
            acc.upload(2, x)
            _say(f"case cooperative {path} pos={pos} rows={rows}")
            rc, _ = acc.task(18, 0, rows, pos, 2, 0)
            assert rc == 0
            got = acc.download(0, rows)
            code, want, _ = om.task((kc, vc), 18, 0, x, pos)
            assert code == 0
            assert first_mismatch(got, want) is None, (pos, rows)
        for h in range(spec.kv_heads):
            k, v = acc.kv_read(0, h, 0, n + 1)
            assert first_mismatch(k, kc[0, h, :n + 1]) is None
            assert first_mismatch(v, vc[0, h, :n + 1]) is None
