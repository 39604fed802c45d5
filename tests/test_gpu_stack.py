"""The persistent decode launch: decode tasks (1-2 rows, Task 18 / 19 / 16)
are collected and run as one launch of resident workgroups that walk every
phase of every sublayer (csrc/decode_stack.hip).  Results must equal the
oracle's whether a launch holds one task (the caller reads the rows after
each) or a whole multi-layer forward; the launch must engage where it
applies; a wait that gives up is reported at the next synchronisation and
the context stays usable; the arrival counters may wrap past 2^32.
"""
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


def _accel(spec, layers, max_seq, env=None):
    import llm_accel
    env = dict(env or {})
    env.setdefault("LLM_ACCEL_STACK", "1")
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


def _oracle_forward(om, kv, layers, h, pos, final=True):
    cur = h
    outs = []
    for layer in range(layers):
        for op in (18, 19):
            code, cur, _ = om.task(kv, op, layer, cur, pos)
            assert code == 0
            outs.append(cur)
    if final:
        _, cur, _ = om.task(kv, 20, 0, cur, pos)
    return outs, cur


def _check_kv(acc, kv, layers, kv_heads, n):
    for layer in range(layers):
        for h in range(kv_heads):
            gk, gv = acc.kv_read(layer, h, 0, n)
            assert np.array_equal(gk, kv[0][layer, h, :n]), ("K", layer, h)
            assert np.array_equal(gv, kv[1][layer, h, :n]), ("V", layer, h)


def test_stack_one_task_per_launch_matches_oracle():
    """Rows read after every task: each launch holds one sublayer."""
    spec = workloads.CONFIG_B
    layers = 1
    synth = workloads.SyntheticModel(spec, layers=layers)
    om = oracle_from_synthetic(synth, oracle_shape(spec, layers=layers, max_seq=64))
    kv = om.new_kv()
    hidden = synth.hidden_rows(12)
    with _accel(spec, layers, 64) as acc:
        acc.load_model(synth)
        for pos, rows in ((0, 8), (8, 1), (9, 2), (11, 1)):
            h = hidden[pos:pos + rows]
            acc.upload(1, h)
            acc.kernel_timing(True)
            cur = h
            for op, pin, pout in ((18, 1, 0), (19, 0, 1), (20, 1, 0)):
                _say(f"case stack single pos={pos} rows={rows} op={op}")
                code, want, ost = om.task(kv, op, 0, cur, pos)
                rc, st = acc.task(op, 0, rows, pos, pin, pout)
                assert rc == 0 and st.as_tuple() == ost.as_tuple()
                err = first_mismatch(acc.download(pout, rows), want)
                assert err is None, f"pos {pos} op {op}: {err}"
                cur = want
            stats = acc.kernel_stats()
            acc.kernel_timing(False)
            if rows <= 2:
                assert stats["decode_stack"][0] == 2, stats
                assert stats["attn_sublayer"][0] == 0 and stats["attention"][0] == 0, stats
            else:
                assert stats["decode_stack"][0] == 0, stats
        _check_kv(acc, kv, layers, spec.kv_heads, 12)


@pytest.mark.parametrize("layers", [2, 4])
def test_stack_whole_forward_in_one_launch(layers):
    """A whole decode forward (T18 / T19 of every layer, then T20) is one
    launch; a prompt block, single rows and row pairs at positions across
    the tile boundaries of the split-head range."""
    spec = workloads.CONFIG_B
    max_seq = 256
    synth = workloads.SyntheticModel(spec, layers=layers)
    om = oracle_from_synthetic(synth, oracle_shape(spec, layers=layers, max_seq=max_seq))
    kv = om.new_kv()
    schedule = [(0, 8)] + [(p, 1) for p in range(8, 62)] + [(62, 2), (64, 1), (65, 2)]
    schedule += [(p, 1) for p in range(67, 127)] + [(127, 2), (129, 1)]
    schedule += [(p, 2) for p in range(130, 254, 2)] + [(254, 1), (255, 1)]
    total = sum(r for _, r in schedule)
    assert total == max_seq
    hidden = synth.hidden_rows(total)
    with _accel(spec, layers, max_seq) as acc:
        acc.load_model(synth)
        acc.kernel_timing(True)
        for pos, rows in schedule:
            h = hidden[pos:pos + rows]
            acc.upload(1, h)
            for layer in range(layers):
                acc.task(18, layer, rows, pos, 1, 0)
                acc.task(19, layer, rows, pos, 0, 1)
            acc.task(20, 0, rows, pos, 1, 0)
            got = acc.download(0, rows)
            _, want = _oracle_forward(om, kv, layers, h, pos)
            err = first_mismatch(got, want)
            assert err is None, f"layers {layers} pos {pos} rows {rows}: {err}"
        stats = acc.kernel_stats()
        acc.kernel_timing(False)
        decode_forwards = sum(1 for _, r in schedule if r <= 2)
        assert stats["decode_stack"][0] == decode_forwards, stats
        _check_kv(acc, kv, layers, spec.kv_heads, max_seq)


def test_stack_mixed_bindings_op16_and_lone_sublayers():
    """Task 16 (both sublayers, in place), a lone FFN sublayer and a lone
    attention sublayer in one run; then the rows are read."""
    spec = workloads.CONFIG_B
    layers = 2
    synth = workloads.SyntheticModel(spec, layers=layers)
    om = oracle_from_synthetic(synth, oracle_shape(spec, layers=layers, max_seq=64))
    kv = om.new_kv()
    hidden = synth.hidden_rows(16)
    with _accel(spec, layers, 64) as acc:
        acc.load_model(synth)
        acc.upload(2, hidden[0:8])
        _, cur, _ = om.task(kv, 16, 0, hidden[0:8], 0)
        _, cur, _ = om.task(kv, 16, 1, cur, 0)
        acc.task(16, 0, 8, 0, 2, 2)
        acc.task(16, 1, 8, 0, 2, 2)
        for pos, rows in ((8, 2), (10, 1)):
            h = hidden[pos:pos + rows]
            acc.upload(3, h)
            _say(f"case stack mixed pos={pos} rows={rows}")
            # op 16 in place on pair 3, then layer 1's attention 3 -> 0 and
            # its FFN 0 -> 0 in place
            acc.task(16, 0, rows, pos, 3, 3)
            acc.task(18, 1, rows, pos, 3, 0)
            acc.task(19, 1, rows, pos, 0, 0)
            _, c1, _ = om.task(kv, 16, 0, h, pos)
            _, c2, _ = om.task(kv, 18, 1, c1, pos)
            _, c3, _ = om.task(kv, 19, 1, c2, pos)
            assert first_mismatch(acc.download(3, rows), c1) is None
            assert first_mismatch(acc.download(0, rows), c3) is None
        _check_kv(acc, kv, layers, spec.kv_heads, 11)


def test_stack_wait_time_out_is_reported_and_cleared():
    """A wait bound of zero ticks makes the launch's waits give up; the
    error is reported at the next synchronisation and the counters are
    cleared, so a context with the normal bound then matches the oracle."""
    import llm_accel
    spec = workloads.CONFIG_B
    layers = 2
    synth = workloads.SyntheticModel(spec, layers=layers)
    hidden = synth.hidden_rows(3)
    with _accel(spec, layers, 64, {"LLM_ACCEL_WAIT_LIMIT": "0"}) as acc:
        acc.load_model(synth)
        acc.upload(1, hidden[0:1])
        for layer in range(layers):
            acc.task(18, layer, 1, 0, 1, 0)
            acc.task(19, layer, 1, 0, 0, 1)
        with pytest.raises(llm_accel.AccelError):
            acc.sync()
        acc.sync()  # cleared: the next synchronisation succeeds


@pytest.mark.parametrize("start", [0, 0xFFFFFF00])
def test_stack_counters_wrap(start):
    """Arrival counters starting just below 2^32 wrap within a few
    launches; results still match the oracle."""
    spec = workloads.CONFIG_B
    layers = 2
    synth = workloads.SyntheticModel(spec, layers=layers)
    om = oracle_from_synthetic(synth, oracle_shape(spec, layers=layers, max_seq=64))
    kv = om.new_kv()
    hidden = synth.hidden_rows(20)
    with _accel(spec, layers, 64, {"LLM_ACCEL_SYNC_START": str(start)}) as acc:
        acc.load_model(synth)
        for pos in range(20):
            h = hidden[pos:pos + 1]
            acc.upload(1, h)
            for layer in range(layers):
                acc.task(18, layer, 1, pos, 1, 0)
                acc.task(19, layer, 1, pos, 0, 1)
            acc.task(20, 0, 1, pos, 1, 0)
            _, want = _oracle_forward(om, kv, layers, h, pos)
            err = first_mismatch(acc.download(0, 1), want)
            assert err is None, f"start {start:#x} pos {pos}: {err}"
