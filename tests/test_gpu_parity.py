"""HIP path vs the CPU oracle, bit-exact: hidden states after every task,
KV-cache contents and status records (reference contract: host
verify-composed-prefill-block / generate --verify-e2e-golden,
host/host_qwen_8x64.cpp:5227-5316, :9144-9249, where the reference
observed max_raw_error 0 at the Qwen shape)."""
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


def _run_sequence(spec, layers, schedule, max_seq, seed=workloads.SEED,
                  check_kv=True):
    """schedule: list of (position, rows) blocks.  Runs T18/T19 per layer and
    T20 on both paths, comparing after every task."""
    import llm_accel
    synth = workloads.SyntheticModel(spec, seed=seed, layers=layers)
    oshape = oracle_shape(spec, layers=layers, max_seq=max_seq)
    om = oracle_from_synthetic(synth, oshape)
    kv = om.new_kv()
    total_rows = sum(r for _, r in schedule)
    hidden_all = synth.hidden_rows(total_rows)
    with llm_accel.Accelerator(accel_shape(spec, layers=layers,
                                           max_seq=max_seq)) as acc:
        acc.load_model(synth)
        row0 = 0
        for pos, rows in schedule:
            h = hidden_all[row0:row0 + rows]
            row0 += rows
            acc.upload(2, h)
            cur = h
            pair_in, pair_out = 2, 0
            for layer in range(layers):
                for op in (18, 19):
                    _say(f"case {spec.name} L{layers} pos={pos} rows={rows} "
                         f"layer={layer} op={op}")
                    code, want, ost = om.task(kv, op, layer, cur, pos)
                    assert code == 0
                    rc, st = acc.task(op, layer, rows, pos, pair_in, pair_out)
                    assert rc == 0
                    got = acc.download(pair_out, rows)
                    assert st.as_tuple() == ost.as_tuple()
                    err = first_mismatch(got, want)
                    assert err is None, f"op {op} layer {layer}: {err}"
                    cur = want
                    pair_in, pair_out = pair_out, pair_in
            _say(f"case {spec.name} pos={pos} rows={rows} op=20")
            code, want, ost = om.task(kv, 20, 0, cur, pos)
            rc, st = acc.task(20, 0, rows, pos, pair_in, pair_out)
            got = acc.download(pair_out, rows)
            assert st.as_tuple() == ost.as_tuple()
            assert first_mismatch(got, want) is None
        if check_kv:
            end = row0
            for layer in range(layers):
                for h in range(spec.kv_heads):
                    k, v = acc.kv_read(layer, h, 0, end)
                    err = first_mismatch(k, kv[0][layer, h, :end])
                    assert err is None, f"K cache layer {layer} head {h}: {err}"
                    err = first_mismatch(v, kv[1][layer, h, :end])
                    assert err is None, f"V cache layer {layer} head {h}: {err}"


def test_config_a_p8_then_decode():
    # one P8 block then two single-row decode forwards.
    _run_sequence(workloads.CONFIG_A, 1, [(0, 8), (8, 1), (9, 1)], max_seq=64)


def test_config_a_two_layers_ragged_blocks():
    # Ragged blocks (R = 3, 5, 8, 1) crossing the 64-position tile edge.
    _run_sequence(workloads.CONFIG_A, 2, [(0, 3), (3, 5), (8, 8), (16, 1)],
                  max_seq=128)


def test_config_a_tile_boundary():
    # A block straddling positions 60..67 exercises two tiles per row.
    spec = workloads.CONFIG_A
    blocks = [(p, 8) for p in range(0, 56, 8)] + [(56, 4), (60, 8), (68, 1)]
    _run_sequence(spec, 1, blocks, max_seq=128)


def test_config_b_p8_then_decode():
    # one Qwen2.5-3B-shaped layer, P8 then one decode.
    _run_sequence(workloads.CONFIG_B, 1, [(0, 8), (8, 1)], max_seq=64)


def test_decoder_layer_op16_matches_18_19():
    import llm_accel
    spec = workloads.CONFIG_A
    synth = workloads.SyntheticModel(spec, layers=1)
    h = synth.hidden_rows(6)
    with llm_accel.Accelerator(accel_shape(spec, layers=1, max_seq=64)) as a:
        a.load_model(synth)
        a.upload(2, h)
        _say("case op16")
        rc, st16 = a.task(16, 0, 6, 0, 2, 0)
        got16 = a.download(0, 6)
        a.kv_clear()
        a.upload(2, h)
        a.task(18, 0, 6, 0, 2, 0)
        a.task(19, 0, 6, 0, 0, 1)
        got = a.download(1, 6)
        assert first_mismatch(got16, got) is None
        oshape = oracle_shape(spec, layers=1, max_seq=64)
        om = oracle_from_synthetic(synth, oshape)
        code, want, ost = om.task(om.new_kv(), 16, 0, h, 0)
        assert code == 0 and rc == 0
        assert st16.as_tuple() == ost.as_tuple()
        # op 16's rows against the oracle's decoder layer (host:4876-4977)
        assert first_mismatch(got16, want) is None


def test_in_place_pairs():
    import llm_accel
    spec = workloads.CONFIG_A
    synth = workloads.SyntheticModel(spec, layers=1)
    h = synth.hidden_rows(4)
    om = oracle_from_synthetic(synth, oracle_shape(spec, layers=1, max_seq=64))
    kv = om.new_kv()
    with llm_accel.Accelerator(accel_shape(spec, layers=1, max_seq=64)) as a:
        a.load_model(synth)
        a.upload(1, h)
        _say("case in-place")
        a.task(18, 0, 4, 0, 1, 1)
        a.task(19, 0, 4, 0, 1, 1)
        a.task(20, 0, 4, 0, 1, 1)
        got = a.download(1, 4)
    _, x, _ = om.task(kv, 18, 0, h, 0)
    _, x, _ = om.task(kv, 19, 0, x, 0)
    _, x, _ = om.task(kv, 20, 0, x, 0)
    assert first_mismatch(got, x) is None


def test_status_validation_matches_controller():
    import llm_accel
    spec = workloads.CONFIG_A
    synth = workloads.SyntheticModel(spec, layers=1)
    om = oracle_from_synthetic(synth, oracle_shape(spec, layers=1, max_seq=64))
    kv = om.new_kv()
    h = synth.hidden_rows(8)
    cases = [
        (18, 0, 9, 0), (18, 0, 0, 0), (21, 0, 1, 0), (5, 0, 1, 0),
        (5, 3, 1, 0), (18, 1, 1, 0), (18, 0, 1, 64), (18, 0, 4, 62),
        (20, 0, 0, 0), (20, 0, 8, 999), (0, 0, 3, 0), (17, 0, 2, 0),
    ]
    with llm_accel.Accelerator(accel_shape(spec, layers=1, max_seq=64)) as a:
        a.load_model(synth)
        a.upload(2, h)
        for op, layer, rows, pos in cases:
            _say(f"case status op={op} layer={layer} rows={rows} pos={pos}")
            rc, st = a.task(op, layer, rows, pos, 2, 0)
            code, _, ost = om.task(kv, op, layer, h[:max(rows, 1)] if rows <= 8
                                   else h, pos, token_count=rows)
            assert rc == code
            assert st.as_tuple() == ost.as_tuple()


def test_kv_preload_then_decode_long_context():
    # BASELINE configs[3] shape at a reduced length: preload K/V, decode one.
    import llm_accel
    spec = workloads.CONFIG_B
    n = 300
    synth = workloads.SyntheticModel(spec, layers=1)
    oshape = oracle_shape(spec, layers=1, max_seq=n + 8)
    om = oracle_from_synthetic(synth, oshape)
    kc, vc = om.new_kv()
    with llm_accel.Accelerator(accel_shape(spec, layers=1, max_seq=n + 8)) as a:
        a.load_model(synth)
        for h in range(spec.kv_heads):
            k, v = synth.kv_rows(n, seed_offset=10 + h)
            kc[0, h, :n] = k
            vc[0, h, :n] = v
            a.kv_write(0, h, 0, k, v)
        x = synth.hidden_rows(1)
        a.upload(2, x)
        _say(f"case preload n={n}")
        a.task(18, 0, 1, n, 2, 0)
        got = a.download(0, 1)
    code, want, _ = om.task((kc, vc), 18, 0, x, n)
    assert first_mismatch(got, want) is None


@pytest.mark.parametrize("n", [128, 1024, 4096, 16384])
def test_context_sweep_decode_forward(n):
    """K/V of one Qwen2.5-3B-shaped layer preloaded
    with seeded Q8.8 N(0, 0.3) to length n, then one decode forward (Task
    18, 19, 20) at position n; every task's output and the appended K/V row
    bit-exact."""
    import llm_accel
    spec = workloads.CONFIG_B
    synth = workloads.SyntheticModel(spec, layers=1)
    oshape = oracle_shape(spec, layers=1, max_seq=n + 64)
    om = oracle_from_synthetic(synth, oshape)
    kc, vc = om.new_kv()
    x = synth.hidden_rows(1)
    with llm_accel.Accelerator(accel_shape(spec, layers=1, max_seq=n + 64)) as a:
        a.load_model(synth)
        for h in range(spec.kv_heads):
            k, v = synth.kv_rows(n, seed_offset=20 + h)
            kc[0, h, :n] = k
            vc[0, h, :n] = v
            a.kv_write(0, h, 0, k, v)
        a.upload(2, x)
        _say(f"case context sweep n={n}")
        got = []
        for op, pin, pout in ((18, 2, 0), (19, 0, 1), (20, 1, 0)):
            rc, st = a.task(op, 0, 1, n, pin, pout)
            assert rc == 0
            got.append(a.download(pout, 1))
        kv_got = [a.kv_read(0, h, n, 1) for h in range(spec.kv_heads)]
    cur = x
    for i, op in enumerate((18, 19, 20)):
        code, cur, _ = om.task((kc, vc), op, 0, cur, n)
        assert code == 0
        err = first_mismatch(got[i], cur)
        assert err is None, f"op {op}: {err}"
    for h in range(spec.kv_heads):
        assert first_mismatch(kv_got[h][0], kc[0, h, n:n + 1]) is None
        assert first_mismatch(kv_got[h][1], vc[0, h, n:n + 1]) is None


@pytest.mark.parametrize("gqa", ["1", "0"])
def test_split_attention_p8_block_late_position(monkeypatch, gqa):
    # 8 rows at positions 500..507: 8-9 tiles per row, split over workgroups
    # (blocks of 3+ rows take the GQA path from 5 tiles; LLM_ACCEL_GQA=0
    # the per-head tile path)
    monkeypatch.setenv("LLM_ACCEL_GQA", gqa)
    import llm_accel
    spec = workloads.CONFIG_A
    n = 500
    synth = workloads.SyntheticModel(spec, layers=1)
    om = oracle_from_synthetic(synth, oracle_shape(spec, layers=1, max_seq=576))
    kc, vc = om.new_kv()
    with llm_accel.Accelerator(accel_shape(spec, layers=1, max_seq=576)) as a:
        a.load_model(synth)
        for h in range(spec.kv_heads):
            k, v = synth.kv_rows(n, seed_offset=20 + h)
            kc[0, h, :n], vc[0, h, :n] = k, v
            a.kv_write(0, h, 0, k, v)
        x = synth.hidden_rows(8)
        a.upload(2, x)
        _say("case split P8 at 500")
        a.task(18, 0, 8, n, 2, 0)
        got = a.download(0, 8)
        kg, vg = a.kv_read(0, 1, 0, n + 8)
    code, want, _ = om.task((kc, vc), 18, 0, x, n)
    assert first_mismatch(got, want) is None
    assert first_mismatch(kg, kc[0, 1, :n + 8]) is None
    assert first_mismatch(vg, vc[0, 1, :n + 8]) is None


@pytest.mark.parametrize("cfg,n,rows", [("B", 1020, 8), ("A", 317, 5), ("B", 256, 1),
                                         ("B", 255, 2), ("B", 252, 8), ("A", 318, 1),
                                         ("A", 382, 1), ("B", 319, 1)])
def test_block_across_tile_boundary_late_context(cfg, n, rows):
    """A block whose rows straddle a 64-position tile boundary after a
    preloaded context, and contexts at the boundary between the
    single-launch (<= 4 tiles) and per-tile attention paths: Task 18
    output rows and every cache row bit-exact."""
    import llm_accel
    spec = workloads.CONFIG_B if cfg == "B" else workloads.CONFIG_A
    synth = workloads.SyntheticModel(spec, layers=1)
    max_seq = n + rows + 64
    om = oracle_from_synthetic(synth, oracle_shape(spec, layers=1, max_seq=max_seq))
    kc, vc = om.new_kv()
    with llm_accel.Accelerator(accel_shape(spec, layers=1, max_seq=max_seq)) as a:
        a.load_model(synth)
        for h in range(spec.kv_heads):
            k, v = synth.kv_rows(n, seed_offset=30 + h)
            kc[0, h, :n], vc[0, h, :n] = k, v
            a.kv_write(0, h, 0, k, v)
        x = synth.hidden_rows(rows, seed_offset=31)
        a.upload(2, x)
        _say(f"case block across tile boundary cfg={cfg} n={n} rows={rows}")
        rc, _ = a.task(18, 0, rows, n, 2, 0)
        assert rc == 0
        got = a.download(0, rows)
        kv_got = [a.kv_read(0, h, 0, n + rows) for h in range(spec.kv_heads)]
    code, want, _ = om.task((kc, vc), 18, 0, x, n)
    assert code == 0
    err = first_mismatch(got, want)
    assert err is None, err
    for h in range(spec.kv_heads):
        assert first_mismatch(kv_got[h][0], kc[0, h, :n + rows]) is None
        assert first_mismatch(kv_got[h][1], vc[0, h, :n + rows]) is None


@pytest.mark.parametrize("n", [40, 150, 700])
def test_saturating_kv_takes_exact_path(n):
    # K/V values beyond +-8.0 saturate in Q4.12; the kernel must switch to
    # the per-product path on those tiles (fused for n=40 and 150, split
    # for 700).
    import llm_accel
    spec = workloads.CONFIG_B
    synth = workloads.SyntheticModel(spec, layers=1)
    om = oracle_from_synthetic(synth, oracle_shape(spec, layers=1, max_seq=n + 8))
    kc, vc = om.new_kv()
    rng = np.random.default_rng(n)
    with llm_accel.Accelerator(accel_shape(spec, layers=1, max_seq=n + 8)) as a:
        a.load_model(synth)
        for h in range(spec.kv_heads):
            k = rng.integers(-9000, 9000, (n, spec.head_dim), dtype=np.int16)
            v = rng.integers(-9000, 9000, (n, spec.head_dim), dtype=np.int16)
            k[: n // 2] //= 8  # first tiles mostly in range
            kc[0, h, :n], vc[0, h, :n] = k, v
            a.kv_write(0, h, 0, k, v)
        x = synth.hidden_rows(2)
        a.upload(2, x)
        _say(f"case saturating kv n={n}")
        a.task(18, 0, 2, n, 2, 0)
        got = a.download(0, 2)
    code, want, _ = om.task((kc, vc), 18, 0, x, n)
    assert first_mismatch(got, want) is None


@pytest.mark.parametrize("cfg,n", [("B", 40), ("B", 700), ("A", 40), ("A", 700)])
def test_saturation_only_outside_first_word(cfg, n):
    """Saturating K / V values (>= 2048, Q4.12 +8.0) only in words 1-3 of
    every bank-paired 8-element group (elements / positions j with
    j % 4 != 0), never in word 0: the per-product correction must be
    detected from any word of a chunk (single-launch and per-tile paths,
    head_dim 128 and 64)."""
    import llm_accel
    spec = workloads.CONFIG_B if cfg == "B" else workloads.CONFIG_A
    d = spec.head_dim
    synth = workloads.SyntheticModel(spec, layers=1)
    om = oracle_from_synthetic(synth, oracle_shape(spec, layers=1, max_seq=n + 8))
    kc, vc = om.new_kv()
    rng = np.random.default_rng(4000 + n)
    elem_hot = (np.arange(d) % 4) != 0
    pos_hot = (np.arange(n) % 4) != 0
    with llm_accel.Accelerator(accel_shape(spec, layers=1, max_seq=n + 8)) as a:
        a.load_model(synth)
        for h in range(spec.kv_heads):
            k = rng.integers(-200, 200, (n, d), dtype=np.int16)
            v = rng.integers(-200, 200, (n, d), dtype=np.int16)
            k[:, elem_hot] = rng.integers(2048, 4000, (n, int(elem_hot.sum())), dtype=np.int16)
            v[pos_hot, :] = rng.integers(2048, 4000, (int(pos_hot.sum()), d), dtype=np.int16)
            kc[0, h, :n], vc[0, h, :n] = k, v
            a.kv_write(0, h, 0, k, v)
        x = synth.hidden_rows(2, seed_offset=41)
        a.upload(2, x)
        _say(f"case saturation outside word 0 cfg={cfg} n={n}")
        a.task(18, 0, 2, n, 2, 0)
        got = a.download(0, 2)
    code, want, _ = om.task((kc, vc), 18, 0, x, n)
    err = first_mismatch(got, want)
    assert err is None, err


def test_accumulator_saturation_over_long_context():
    # K = 0 (every score 0, uniform probabilities) and V saturated at +8.0
    # over 16384 positions: the attention accumulator reaches the Q16.16
    # bound, so chunks of the split scan must fall back to the per-tile
    # saturating recurrence.
    import llm_accel
    spec = workloads.CONFIG_B
    n = 16384
    synth = workloads.SyntheticModel(spec, layers=1)
    om = oracle_from_synthetic(synth, oracle_shape(spec, layers=1, max_seq=n + 64))
    kc, vc = om.new_kv()
    x = synth.hidden_rows(1)
    with llm_accel.Accelerator(accel_shape(spec, layers=1, max_seq=n + 64)) as a:
        a.load_model(synth)
        for h in range(spec.kv_heads):
            k = np.zeros((n, spec.head_dim), np.int16)
            v = np.full((n, spec.head_dim), 32767, np.int16)
            kc[0, h, :n], vc[0, h, :n] = k, v
            a.kv_write(0, h, 0, k, v)
        a.upload(2, x)
        _say("case accumulator saturation n=16384")
        a.task(18, 0, 1, n, 2, 0)
        got = a.download(0, 1)
    code, want, _ = om.task((kc, vc), 18, 0, x, n)
    assert first_mismatch(got, want) is None


@pytest.mark.parametrize("n,period", [(16384, 1), (16384, 10), (4096, 3)])
def test_running_max_rises_often(n, period):
    """K rows of tile j are a fixed +-8 raw pattern times 1 + j // period:
    for query heads whose score along the pattern is positive the tile
    maxima rise every `period` tiles (257 rises at period 1 -- the tile-by-
    tile recurrence -- and about 26 at period 10, each a separate run of
    the parallel one), up to K values past the Q4.12 bound (the saturation
    correction); decode row and KV against the oracle."""
    import llm_accel
    spec = workloads.CONFIG_B
    synth = workloads.SyntheticModel(spec, layers=1)
    om = oracle_from_synthetic(synth, oracle_shape(spec, layers=1, max_seq=n + 64))
    kc, vc = om.new_kv()
    rng = np.random.default_rng(9000 + period)
    x = synth.hidden_rows(1, seed_offset=51)
    with llm_accel.Accelerator(accel_shape(spec, layers=1, max_seq=n + 64)) as a:
        a.load_model(synth)
        for h in range(spec.kv_heads):
            u = rng.choice(np.array([-8, 8], np.int16), spec.head_dim)
            step = 1 + (np.arange(n) // 64) // period
            k = np.clip(step[:, None].astype(np.int64) * u[None, :], -32768, 32767)
            k = k.astype(np.int16)
            _, v = synth.kv_rows(n, seed_offset=60 + h)
            kc[0, h, :n], vc[0, h, :n] = k, v
            a.kv_write(0, h, 0, k, v)
        a.upload(2, x)
        _say(f"case running max rises n={n} period={period}")
        rc, _ = a.task(18, 0, 1, n, 2, 0)
        assert rc == 0
        got = a.download(0, 1)
        kv_got = [a.kv_read(0, h, n, 1) for h in range(spec.kv_heads)]
    code, want, _ = om.task((kc, vc), 18, 0, x, n)
    assert code == 0
    err = first_mismatch(got, want)
    assert err is None, err
    for h in range(spec.kv_heads):
        assert first_mismatch(kv_got[h][0], kc[0, h, n:n + 1]) is None
        assert first_mismatch(kv_got[h][1], vc[0, h, n:n + 1]) is None


@pytest.mark.parametrize("cfg,n,rows", [("B", 1024, 1), ("B", 1150, 2), ("A", 4030, 2),
                                         ("B", 4031, 1), ("A", 300, 1), ("B", 2047, 2)])
def test_tile_path_one_launch(cfg, n, rows):
    """Decode rows at 5-63 tiles take the tile path in one launch (tile
    maxima exchanged between the workgroups of the launch); up to 63
    tiles, both head_dims, blocks across a tile boundary."""
    test_block_across_tile_boundary_late_context(cfg, n, rows)


@pytest.mark.parametrize("cfg,n,rows", [("B", 16447, 1), ("B", 16448, 1), ("B", 16446, 2),
                                         ("A", 16447, 1)])
def test_gqa_one_launch_tile_limit(cfg, n, rows):
    """The GQA path at the one-launch limit: 257 tiles with one row (scores,
    PV and scan in one launch), 258 tiles (three launches), 257 tiles with
    two rows (a grid past what the device holds at once: separate
    launches); both head_dims."""
    test_block_across_tile_boundary_late_context(cfg, n, rows)


@pytest.fixture
def tile_two_launches(monkeypatch):
    """The tile path as two launches (scores, then PV and recurrence)."""
    monkeypatch.setenv("LLM_ACCEL_TILE_FUSED", "0")


@pytest.mark.parametrize("cfg,n,rows", [("B", 1024, 1), ("A", 382, 1), ("B", 255, 2),
                                         ("A", 4030, 2)])
def test_tile_path_two_launches(tile_two_launches, cfg, n, rows):
    test_block_across_tile_boundary_late_context(cfg, n, rows)


@pytest.mark.parametrize("cfg,n,rows", [("B", 1020, 8), ("A", 317, 5), ("B", 252, 8),
                                         ("A", 700, 3)])
def test_tile_path_multirow_blocks(monkeypatch, cfg, n, rows):
    # blocks of 3+ rows take the GQA path from 5 tiles by default; with it
    # off they run the per-head tile path (one launch when the grid fits,
    # else two)
    monkeypatch.setenv("LLM_ACCEL_GQA", "0")
    test_block_across_tile_boundary_late_context(cfg, n, rows)


def test_tile_path_one_launch_running_max_rises(monkeypatch):
    # every tile raises the running max (the recurrence's rescaling path)
    monkeypatch.setenv("LLM_ACCEL_GQA_MIN_TILES", "1000")
    test_running_max_rises_often(2048, 1)


@pytest.fixture
def gqa_everywhere(monkeypatch):
    """Contexts of 5 tiles and more take the GQA tile path (by default it
    starts at 64 tiles, where it overtakes the per-head path)."""
    monkeypatch.setenv("LLM_ACCEL_GQA_MIN_TILES", "5")


@pytest.mark.parametrize("cfg,n,rows", [("B", 1020, 8), ("A", 317, 5), ("B", 319, 1),
                                         ("A", 382, 1), ("B", 255, 2)])
def test_gqa_path_block_across_tile_boundary(gqa_everywhere, cfg, n, rows):
    """The GQA tile path (head_dim 128 and 64) on blocks that straddle a
    tile boundary after a preloaded context."""
    test_block_across_tile_boundary_late_context(cfg, n, rows)


@pytest.mark.parametrize("cfg,n", [("B", 700), ("A", 700)])
def test_gqa_path_saturation(gqa_everywhere, cfg, n):
    test_saturation_only_outside_first_word(cfg, n)


def test_gqa_path_saturating_kv(gqa_everywhere):
    test_saturating_kv_takes_exact_path(700)


def test_gqa_path_running_max_rises(gqa_everywhere):
    test_running_max_rises_often(4096, 3)


@pytest.fixture
def gqa_three_launches(monkeypatch):
    """The GQA tile path from 5 tiles as three launches (scores, PV, scan)
    instead of scores and PV in one launch."""
    monkeypatch.setenv("LLM_ACCEL_GQA_MIN_TILES", "5")
    monkeypatch.setenv("LLM_ACCEL_GQA_FUSED", "0")


@pytest.mark.parametrize("cfg,n,rows", [("B", 1020, 8), ("A", 317, 5), ("B", 319, 1)])
def test_gqa_three_launches_block_across_tile_boundary(gqa_three_launches, cfg, n, rows):
    test_block_across_tile_boundary_late_context(cfg, n, rows)


def test_gqa_three_launches_running_max_rises(gqa_three_launches):
    test_running_max_rises_often(4096, 3)


@pytest.mark.parametrize("scan_fused", ["1", "0"])
def test_gqa_epoch_wraps(monkeypatch, scan_fused):
    """The GQA path's launch epoch started just below its maximum: six
    decode rows in a row (5-6 tiles, the GQA path forced from 5 tiles), the
    fourth launch past the maximum clears the tagged maxima and sums and
    starts again at 1; every row and K/V append against the oracle."""
    import llm_accel
    monkeypatch.setenv("LLM_ACCEL_GQA_MIN_TILES", "5")
    monkeypatch.setenv("LLM_ACCEL_GQA_EPOCH_START", "65532")
    monkeypatch.setenv("LLM_ACCEL_GQA_SCAN_FUSED", scan_fused)
    spec = workloads.CONFIG_B
    synth = workloads.SyntheticModel(spec, layers=1)
    n0 = 317
    om = oracle_from_synthetic(synth, oracle_shape(spec, layers=1, max_seq=n0 + 16))
    kc, vc = om.new_kv()
    xs = synth.hidden_rows(6, seed_offset=77)
    with llm_accel.Accelerator(accel_shape(spec, layers=1, max_seq=n0 + 16)) as a:
        a.load_model(synth)
        for h in range(spec.kv_heads):
            k, v = synth.kv_rows(n0, seed_offset=30 + h)
            kc[0, h, :n0], vc[0, h, :n0] = k, v
            a.kv_write(0, h, 0, k, v)
        for i in range(6):
            pos = n0 + i
            _say(f"case epoch wrap scan_fused={scan_fused} pos={pos}")
            a.upload(2, xs[i:i + 1])
            rc, _ = a.task(18, 0, 1, pos, 2, 0)
            assert rc == 0
            got = a.download(0, 1)
            code, want, _ = om.task((kc, vc), 18, 0, xs[i:i + 1], pos)
            assert code == 0
            err = first_mismatch(got, want)
            assert err is None, f"pos {pos}: {err}"
        for h in range(spec.kv_heads):
            k, v = a.kv_read(0, h, n0, 6)
            assert first_mismatch(k, kc[0, h, n0:n0 + 6]) is None
            assert first_mismatch(v, vc[0, h, n0:n0 + 6]) is None


def test_gqa_epoch_wrap_clears_stale_words(monkeypatch):
    """A full epoch period in one context: a decode row at 700 positions
    (11 tiles) leaves maxima and sums tagged with epoch 1 at tiles 0-10;
    65,534 decode rows at position 320 (6 tiles) retag tiles 0-5 only;
    the next launch wraps to epoch 1 and runs over 11 tiles again with
    another row, where tiles 6-10 still hold the first row's epoch-1
    words unless the wrap cleared them.  Both rows and the appended K/V
    are checked against the oracle."""
    import llm_accel
    monkeypatch.setenv("LLM_ACCEL_GQA_MIN_TILES", "5")
    spec = workloads.CONFIG_A
    synth = workloads.SyntheticModel(spec, layers=1)
    n0, filler_pos = 700, 320
    om = oracle_from_synthetic(synth, oracle_shape(spec, layers=1, max_seq=n0 + 8))
    kc, vc = om.new_kv()
    xs = synth.hidden_rows(3, seed_offset=91)
    with llm_accel.Accelerator(accel_shape(spec, layers=1, max_seq=n0 + 8)) as a:
        a.load_model(synth)
        for h in range(spec.kv_heads):
            k, v = synth.kv_rows(n0, seed_offset=50 + h)
            kc[0, h, :n0], vc[0, h, :n0] = k, v
            a.kv_write(0, h, 0, k, v)
        _say("case epoch period: first row at 700 (epoch 1)")
        a.upload(2, xs[0:1])
        assert a.task(18, 0, 1, n0, 2, 0)[0] == 0
        got = a.download(0, 1)
        _, want, _ = om.task((kc, vc), 18, 0, xs[0:1], n0)
        assert first_mismatch(got, want) is None
        _say("case epoch period: 65,534 rows at 320 (epochs 2..65535)")
        a.upload(3, xs[1:2])
        for i in range(65534):
            rc, _ = a.task(18, 0, 1, filler_pos, 3, 1)
            assert rc == 0, i
        got = a.download(1, 1)
        _, want, _ = om.task((kc, vc), 18, 0, xs[1:2], filler_pos)
        assert first_mismatch(got, want) is None
        _say("case epoch period: wrap to epoch 1 at 700 with another row")
        a.upload(2, xs[2:3])
        assert a.task(18, 0, 1, n0, 2, 0)[0] == 0
        got = a.download(0, 1)
        _, want, _ = om.task((kc, vc), 18, 0, xs[2:3], n0)
        assert first_mismatch(got, want) is None
        for h in range(spec.kv_heads):
            k, v = a.kv_read(0, h, 0, n0 + 1)
            assert first_mismatch(k, kc[0, h, :n0 + 1]) is None
            assert first_mismatch(v, vc[0, h, :n0 + 1]) is None


@pytest.fixture
def gqa_scan_launch(monkeypatch):
    """The GQA tile path from 5 tiles with scores and PV in one launch and
    the scan as a launch of its own (by default the scan's workgroups run
    in the same launch, reading the tiles' tagged sums)."""
    monkeypatch.setenv("LLM_ACCEL_GQA_MIN_TILES", "5")
    monkeypatch.setenv("LLM_ACCEL_GQA_SCAN_FUSED", "0")


@pytest.mark.parametrize("cfg,n,rows", [("B", 1020, 8), ("A", 317, 5), ("B", 319, 1)])
def test_gqa_scan_launch_block_across_tile_boundary(gqa_scan_launch, cfg, n, rows):
    test_block_across_tile_boundary_late_context(cfg, n, rows)


def test_gqa_scan_launch_running_max_rises(gqa_scan_launch):
    test_running_max_rises_often(16384, 10)


def test_norm_cache_invalidation():
    # T18 writes pair 0 and derives its FFN norm; uploading new rows into
    # pair 0 before T19 must discard that copy.  T19 into pair 1 derives the
    # next layer's attention norm; T18 on a different pair must not use it.
    import llm_accel
    spec = workloads.CONFIG_A
    synth = workloads.SyntheticModel(spec, layers=2)
    om = oracle_from_synthetic(synth, oracle_shape(spec, layers=2, max_seq=64))
    kv = om.new_kv()
    h = synth.hidden_rows(12)
    with llm_accel.Accelerator(accel_shape(spec, layers=2, max_seq=64)) as a:
        a.load_model(synth)
        a.upload(2, h[:4])
        a.task(18, 0, 4, 0, 2, 0)
        a.upload(0, h[4:8])           # overwrite T18's output
        a.task(19, 0, 4, 0, 0, 1)
        got19 = a.download(1, 4)
        a.upload(3, h[8:12])
        a.task(18, 1, 4, 0, 3, 2)     # layer 1 on a pair T19 did not write
        got18 = a.download(2, 4)
        _say("case norm cache")
    _, _, _ = om.task(kv, 18, 0, h[:4], 0)
    _, want19, _ = om.task(kv, 19, 0, h[4:8], 0)
    _, want18, _ = om.task(kv, 18, 1, h[8:12], 0)
    assert first_mismatch(got19, want19) is None
    assert first_mismatch(got18, want18) is None


def test_final_norm_rows_beyond_token_count_unchanged():
    # Task 20 writes rows < token_count of its output pair and leaves the
    # other rows as they were, whichever way the library produces it
    # (buffer exchange after the last layer's FFN, or the norm kernel when
    # the row count differs or the pair's address was handed out).
    import llm_accel
    spec = workloads.CONFIG_A
    layers = 2
    synth = workloads.SyntheticModel(spec, layers=layers)
    om = oracle_from_synthetic(synth, oracle_shape(spec, layers=layers, max_seq=64))
    kv = om.new_kv()
    h = synth.hidden_rows(15)
    final_gamma = synth.norms()[2 * layers]

    def forward(a, x, rows, pos):
        a.upload(1, x)
        for layer in range(layers):
            a.task(18, layer, rows, pos, 1, 0)
            a.task(19, layer, rows, pos, 0, 1)

    def oracle_forward(x, pos):
        for layer in range(layers):
            _, x, _ = om.task(kv, 18, layer, x, pos)
            _, x, _ = om.task(kv, 19, layer, x, pos)
        return x

    with llm_accel.Accelerator(accel_shape(spec, layers=layers, max_seq=64)) as a:
        a.load_model(synth)
        _say("case final norm exchange P8")
        forward(a, h[:8], 8, 0)
        a.task(20, 0, 8, 0, 1, 0)
        got8 = a.download(0, 8)
        x8 = oracle_forward(h[:8], 0)
        assert first_mismatch(got8, orc.rmsnorm(x8, final_gamma)) is None
        _say("case final norm exchange decode")
        forward(a, h[8:9], 1, 8)
        before = a.download(0, 8)
        a.task(20, 0, 1, 8, 1, 0)
        after = a.download(0, 8)
        x9 = oracle_forward(h[8:9], 8)
        assert first_mismatch(after[:1], orc.rmsnorm(x9, final_gamma)) is None
        assert first_mismatch(after[1:], before[1:]) is None
        _say("case final norm row-count mismatch")
        forward(a, h[9:12], 3, 9)
        before = a.download(0, 8)
        a.task(20, 0, 2, 9, 1, 0)
        after = a.download(0, 8)
        x12 = oracle_forward(h[9:12], 9)
        assert first_mismatch(after[:2], orc.rmsnorm(x12[:2], final_gamma)) is None
        assert first_mismatch(after[2:], before[2:]) is None
        _say("case final norm exported pair")
        ptr = llm_accel.lib().llm_pair_device_ptr(a._ctx, 0)
        assert ptr
        forward(a, h[12:15], 3, 12)
        a.task(20, 0, 3, 12, 1, 0)
        assert llm_accel.lib().llm_pair_device_ptr(a._ctx, 0) == ptr
        after = a.download(0, 3)
        x15 = oracle_forward(h[12:15], 12)
        assert first_mismatch(after, orc.rmsnorm(x15, final_gamma)) is None
