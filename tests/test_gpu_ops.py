"""Operator-level commands (ops 1-15, 17) on the HIP path vs the CPU oracle,
bit-exact, plus their status records and rejections.

Mirrors the reference host's operator checks: run_random_verification
(host/host_qwen_8x64.cpp:3812-4163: projections, residual, RMSNorm,
SiLU*up, QK / PV over a 13-position tile, DECODE_SMOKE over two steps),
run_decode_smoke_verification (:4166-4265) and the prefill attention block
profile (:5578-5625, its task / packet counts).  The reference compares
with tolerances (1 raw for projections / norms / QK / PV, 4 for flash
attention) because its goldens are separate from the FPGA datapath; here
the oracle restates those goldens and the HIP path must equal them.
"""
import sys

import numpy as np
import pytest

from oracle import orc
import workloads
from helpers import accel_shape, first_mismatch

pytestmark = pytest.mark.gpu

# configs[0]'s shape with room for positions past one tile, and configs[1]'s
CONFIG_A_OPS = workloads.with_layers(workloads.CONFIG_A, 1, max_seq=256)
CONFIG_B_SHORT = workloads.with_layers(workloads.CONFIG_B, 1, max_seq=2048)
SPECS = [CONFIG_A_OPS, CONFIG_B_SHORT]


def _say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def _ints(rng, shape, lo, hi):
    return rng.integers(lo, hi + 1, size=shape).astype(np.int16)


@pytest.fixture(scope="module", params=SPECS, ids=lambda s: s.name)
def ctx(request):
    import llm_accel
    spec = request.param
    synth = workloads.SyntheticModel(spec, layers=1)
    acc = llm_accel.Accelerator(accel_shape(spec, layers=1))
    acc.load_model(synth)
    yield spec, synth, acc
    acc.close()


def _group(spec):
    return spec.heads // spec.kv_heads


# ---- ops 1-7: projections ----------------------------------------------------
@pytest.mark.parametrize("rows", [1, 2, 5, 8])
def test_projections_match_oracle(ctx, rows):
    import llm_accel
    spec, synth, acc = ctx
    rng = np.random.default_rng(100 + rows)
    for proj in range(7):
        op = llm_accel.OP_Q_PROJECTION + proj
        out_dim, in_dim = spec.proj_dims(proj)
        x = _ints(rng, (rows, in_dim), -1200, 1200)
        _say(f"case {spec.name} op={op} rows={rows}")
        got = acc.run_feature(op, x)
        want = orc.projection(x, synth.weight(0, proj))
        err = first_mismatch(got, want)
        assert err is None, f"projection op {op}: {err}"


@pytest.mark.parametrize("rows", [1, 2, 5, 8])
def test_projections_with_sparse_corrections(rows):
    """Every projection with a few weights past 12 bits per matrix (at most
    four in a row): the 12-bit images hold them clamped and the corrections
    of their rows add the difference -- K and V as row ranges of the
    Q|K|V matrix, so their corrections sit at an offset -- bit-exact
    against the oracle's full-range projection."""
    import llm_accel
    spec = CONFIG_A_OPS
    synth = workloads.SyntheticModel(spec, layers=1)
    rng = np.random.default_rng(300 + rows)
    for proj in range(7):
        w = synth.weight(0, proj)
        n, k = w.shape
        for r in (0, n // 2, n - 1):
            cols = rng.choice(k, size=4, replace=False)
            w[r, cols] = rng.choice([-32768, -2049, 2048, 30000], size=4)
    with llm_accel.Accelerator(accel_shape(spec, layers=1)) as acc:
        acc.load_model(synth)
        assert acc.weight_bytes()[1] == 0  # every matrix still in 12 bits
        for proj in range(7):
            op = llm_accel.OP_Q_PROJECTION + proj
            out_dim, in_dim = spec.proj_dims(proj)
            x = _ints(rng, (rows, in_dim), -32768, 32767)
            _say(f"case corrections op={op} rows={rows}")
            got = acc.run_feature(op, x)
            want = orc.projection(x, synth.weight(0, proj))
            err = first_mismatch(got, want)
            assert err is None, f"projection op {op}: {err}"


def test_projection_saturates_and_full_range(ctx):
    import llm_accel
    spec, synth, acc = ctx
    rng = np.random.default_rng(7)
    x = _ints(rng, (3, spec.hidden), -32768, 32767)
    got = acc.run_feature(llm_accel.OP_Q_PROJECTION, x)
    assert np.array_equal(got, orc.projection(x, synth.weight(0, 0)))
    assert (np.abs(got.astype(np.int32)) == 32767).any() or (got == -32768).any()


# ---- ops 8-10: vector operators -----------------------------------------------
@pytest.mark.parametrize("rows", [1, 4, 5, 8])
def test_vector_operators_match_oracle(ctx, rows):
    import llm_accel
    spec, synth, acc = ctx
    rng = np.random.default_rng(200 + rows)
    h, i = spec.hidden, spec.inter
    x = _ints(rng, (rows, h), -3000, 3000)
    gamma = _ints(rng, (1, h), 64, 512)
    _say(f"case {spec.name} rmsnorm rows={rows}")
    got = acc.run_feature(llm_accel.OP_RMSNORM, x, gamma)
    assert first_mismatch(got, orc.rmsnorm(x, gamma[0])) is None
    g = _ints(rng, (rows, i), -2600, 2600)
    u = _ints(rng, (rows, i), -4000, 4000)
    _say(f"case {spec.name} silu_mul rows={rows}")
    got = acc.run_feature(llm_accel.OP_SILU_MUL, g, u)
    assert first_mismatch(got, orc.silu_mul(g, u)) is None
    a = _ints(rng, (rows, h), -32768, 32767)
    b = _ints(rng, (rows, h), -32768, 32767)
    _say(f"case {spec.name} residual rows={rows}")
    got = acc.run_feature(llm_accel.OP_RESIDUAL_ADD, a, b)
    assert np.array_equal(got, orc.residual(a, b))


# ---- ops 11-13: one attention tile ---------------------------------------------
@pytest.mark.parametrize("tile_len", [1, 13, 64])
def test_attention_tile_operators_match_oracle(ctx, tile_len):
    import llm_accel
    spec, synth, acc = ctx
    g, d, hk = _group(spec), spec.head_dim, spec.kv_heads
    rng = np.random.default_rng(300 + tile_len)
    q = _ints(rng, (hk, g, d), -96 * 16, 96 * 16)
    k = _ints(rng, (hk, tile_len, d), -96 * 16, 96 * 16)
    k[0, 0, :4] = 4000  # values that saturate in Q4.12
    _say(f"case {spec.name} qk tile_len={tile_len}")
    got, st = acc.run_attention(llm_accel.OP_ATTN_QK, q, k, tile_len=tile_len)
    for h in range(hk):
        want = np.zeros((g, 64), np.int16)
        want[:, :tile_len] = orc.qk_scores(q[h], k[h])
        assert first_mismatch(got[h], want) is None, f"QK head {h}"
    assert (st.output_waves, st.mm_tasks, st.completed_packets) == (1, 2, 64)

    p = _ints(rng, (hk, g, 64), 0, 24 * 16)
    v = _ints(rng, (hk, tile_len, d), -96 * 16, 96 * 16)
    v[-1, -1, :3] = -5000
    _say(f"case {spec.name} pv tile_len={tile_len}")
    got, st = acc.run_attention(llm_accel.OP_ATTN_PV, p, v, tile_len=tile_len)
    for h in range(hk):
        assert first_mismatch(got[h], orc.attention_pv(p[h], v[h])) is None, f"PV head {h}"
    waves = -(-d // 64)
    assert (st.output_waves, st.mm_tasks, st.completed_packets) == (waves, 2 * waves,
                                                                    64 * waves)

    x = _ints(rng, (hk, g, 64), -2500, 2500)
    x[0, 0, :tile_len] = 77  # an all-equal row
    _say(f"case {spec.name} softmax tile_len={tile_len}")
    got, st = acc.run_attention(llm_accel.OP_SOFTMAX, x, tile_len=tile_len)
    for h in range(hk):
        assert first_mismatch(got[h], orc.softmax_rows(x[h], tile_len)) is None
    assert st.vector_tasks == 2 and st.completed_packets == 2 * g * -(-tile_len // 16)


# ---- ops 14 / 15: flash attention of one decode position ------------------------
def _preload(acc, spec, n, seed):
    rng = np.random.default_rng(seed)
    d = spec.head_dim
    ks, vs = [], []
    for h in range(spec.kv_heads):
        k = _ints(rng, (n, d), -48 * 16, 48 * 16)
        v = _ints(rng, (n, d), -48 * 16, 48 * 16)
        acc.kv_write(0, h, 0, k, v)
        ks.append(k)
        vs.append(v)
    return ks, vs


@pytest.mark.parametrize("position", [0, 37, 63, 64, 130])
def test_attention_flash_matches_oracle(ctx, position):
    import llm_accel
    spec, synth, acc = ctx
    if position >= spec.max_seq:
        pytest.skip("beyond the shape's max_seq")
    g, d, hk = _group(spec), spec.head_dim, spec.kv_heads
    ks, vs = _preload(acc, spec, position + 1, 400 + position)
    rng = np.random.default_rng(500 + position)
    q = _ints(rng, (hk, g, d), -48 * 16, 48 * 16)
    _say(f"case {spec.name} flash position={position}")
    got, st = acc.run_attention(llm_accel.OP_ATTN_FLASH, q, position=position)
    for h in range(hk):
        want = orc.attention(q[h], ks[h], vs[h], orc.SEM_LEGACY_Q8_8)
        assert first_mismatch(got[h], want) is None, f"head {h}"
    tiles, waves = -(-(position + 1) // 64), -(-d // 64)
    assert st.mm_tasks == 2 * tiles * (1 + waves)
    assert st.completed_packets == 32 * st.mm_tasks and st.output_waves == waves


def test_attention_flash_long_context():
    import llm_accel
    spec = CONFIG_B_SHORT
    synth = workloads.SyntheticModel(spec, layers=1)
    position = 1500
    with llm_accel.Accelerator(accel_shape(spec, layers=1)) as acc:
        acc.load_model(synth)
        ks, vs = _preload(acc, spec, position + 1, 41)
        g, d, hk = _group(spec), spec.head_dim, spec.kv_heads
        q = _ints(np.random.default_rng(42), (hk, g, d), -48 * 16, 48 * 16)
        _say(f"case {spec.name} flash position={position}")
        got, _ = acc.run_attention(llm_accel.OP_ATTN_FLASH, q, position=position)
        for h in range(hk):
            want = orc.attention(q[h], ks[h], vs[h], orc.SEM_LEGACY_Q8_8)
            assert first_mismatch(got[h], want) is None, f"head {h}"


def test_decode_smoke_steps_append_and_attend(ctx):
    # The reference's random verification: per step, K / V of every KV head
    # arrive in the aux ports, are written at `position`, and the group's
    # queries attend over [0, position].
    import llm_accel
    spec, synth, acc = ctx
    g, d, hk = _group(spec), spec.head_dim, spec.kv_heads
    acc.kv_clear()
    rng = np.random.default_rng(600)
    kc = [np.zeros((0, d), np.int16) for _ in range(hk)]
    vc = [np.zeros((0, d), np.int16) for _ in range(hk)]
    for step in range(3):
        q = _ints(rng, (hk, g, d), -48 * 16, 48 * 16)
        k = _ints(rng, (hk, d), -48 * 16, 48 * 16)
        v = _ints(rng, (hk, d), -48 * 16, 48 * 16)
        _say(f"case {spec.name} decode_smoke step={step}")
        got, st = acc.run_attention(llm_accel.OP_DECODE_SMOKE, q, (k, v),
                                    position=step)
        for h in range(hk):
            kc[h] = np.vstack([kc[h], k[h:h + 1]])
            vc[h] = np.vstack([vc[h], v[h:h + 1]])
            want = orc.attention(q[h], kc[h], vc[h], orc.SEM_LEGACY_Q8_8)
            assert first_mismatch(got[h], want) is None, f"step {step} head {h}"
        assert st.code == 0 and st.op == llm_accel.OP_DECODE_SMOKE
    for h in range(hk):
        kr, vr = acc.kv_read(0, h, 0, 3)
        assert np.array_equal(kr, kc[h]) and np.array_equal(vr, vc[h])


# ---- op 17: prefill attention block ----------------------------------------------
@pytest.mark.parametrize("position,tokens", [(0, 1), (0, 8), (60, 5), (130, 8), (63, 2)])
def test_prefill_attention_block_matches_oracle(ctx, position, tokens):
    import llm_accel
    spec, synth, acc = ctx
    if position + tokens > spec.max_seq:
        pytest.skip("beyond the shape's max_seq")
    g, d, hk = _group(spec), spec.head_dim, spec.kv_heads
    ks, vs = _preload(acc, spec, position + tokens, 700 + position)
    rng = np.random.default_rng(800 + position + tokens)
    q = _ints(rng, (hk, tokens, g, d), -48 * 16, 48 * 16)
    _say(f"case {spec.name} prefill_block position={position} tokens={tokens}")
    got, st = acc.run_prefill_attention_block(q, position, tokens)
    for h in range(hk):
        for t in range(tokens):
            n = position + t + 1
            want = orc.attention(q[h, t], ks[h][:n], vs[h][:n])
            assert first_mismatch(got[h, t], want) is None, f"head {h} token {t}"
    # run_prefill_attention_block's expectations (host:5595-5605)
    tiles, waves = -(-(position + tokens) // 64), -(-d // 64)
    assert st.output_waves == waves
    assert st.mm_tasks == 2 * tiles * g * (1 + waves)
    assert st.completed_packets == 32 * st.mm_tasks


# ---- status records, rejections, explicit device pointers -------------------------
def test_feature_status_counters(ctx):
    import llm_accel
    spec, synth, acc = ctx
    h, i, c = spec.hidden, spec.inter, spec.kv_channels
    for rows in (3, 6):
        for proj in range(7):
            out_dim = spec.proj_dims(proj)[0]
            _, st = acc.op(llm_accel.OP_Q_PROJECTION + proj, 0, rows, 0, 0,
                           np.zeros((rows, spec.proj_dims(proj)[1]), np.int16))
            w = -(-out_dim // 128)
            assert st.as_tuple() == (proj + 1, 0, rows, w, 2 * w, 0, 64 * w, 1)
        for op, dim in ((llm_accel.OP_RMSNORM, h), (llm_accel.OP_SILU_MUL, i),
                        (llm_accel.OP_RESIDUAL_ADD, h)):
            _, st = acc.op(op, 0, rows, 0, 0)
            vt = 1 + (rows > 4)
            assert st.as_tuple() == (op, 0, rows, 0, 0, vt, rows * -(-dim // 16), 1)
    assert c > 0


def test_rejections_follow_the_controller(ctx):
    import llm_accel
    spec, synth, acc = ctx
    g = _group(spec)
    S = llm_accel
    cases = [
        # (op, layer, token_count, position, tile_len) -> (status op, code)
        ((S.OP_Q_PROJECTION, 0, 9, 0, 0), (0, S.BAD_TOKEN_COUNT)),
        ((21, 0, 1, 0, 0), (21, S.BAD_OPERATOR)),
        ((S.OP_NOP, 0, 0, 0, 0), (0, S.STATUS_OK)),
        ((S.OP_RMSNORM, 1, 1, 0, 0), (S.OP_RMSNORM, S.BAD_LAYER)),
        ((S.OP_ATTN_QK, 0, g, 0, 0), (S.OP_ATTN_QK, S.BAD_TILE_LENGTH)),
        ((S.OP_SOFTMAX, 0, g, 0, 65), (S.OP_SOFTMAX, S.BAD_TILE_LENGTH)),
        ((S.OP_ATTN_FLASH, 0, g - 1, 0, 1), (S.OP_ATTN_FLASH, S.BAD_TOKEN_COUNT)),
        ((S.OP_ATTN_FLASH, 0, g, spec.max_seq, 1), (S.OP_ATTN_FLASH, S.BAD_POSITION)),
        ((S.OP_DECODE_SMOKE, 0, g, 0, 65), (S.OP_DECODE_SMOKE, S.BAD_TILE_LENGTH)),
        ((S.OP_ATTN_PREFILL_BLOCK, 0, 0, 0, 0), (S.OP_ATTN_PREFILL_BLOCK,
                                                 S.BAD_TOKEN_COUNT)),
        ((S.OP_ATTN_PREFILL_BLOCK, 0, 4, spec.max_seq - 3, 0),
         (S.OP_ATTN_PREFILL_BLOCK, S.BAD_POSITION)),
        # profile flags in the upper token_count bits are stripped when
        # tile_len != 0 (ctrl:5882-5886)
        ((S.OP_ATTN_QK, 0, (5 << 16) | 9, 0, 13), (0, S.BAD_TOKEN_COUNT)),
    ]
    for args, (sop, code) in cases:
        _, st = acc.op(*args)
        assert (st.op, st.code) == (sop, code), args
    for bad in ((S.OP_DECODER_LAYER, 0, 1, 0, 0), (S.OP_FFN, 0, 1, 0, 0),
                (S.OP_Q_PROJECTION, 0, 1, 0, 3)):
        with pytest.raises(S.AccelError):
            acc.op(*bad)


def test_explicit_device_pointers(ctx):
    import llm_accel
    spec, synth, acc = ctx
    rng = np.random.default_rng(900)
    a = _ints(rng, (4, spec.hidden), -20000, 20000)
    b = _ints(rng, (4, spec.hidden), -20000, 20000)
    acc.port_write(llm_accel.PORT_OUT, a)   # inputs in the out and in ports,
    acc.port_write(llm_accel.PORT_IN, b)    # result into the aux port
    p_in, n = acc.port(llm_accel.PORT_IN)
    p_aux, _ = acc.port(llm_accel.PORT_AUX)
    p_out, _ = acc.port(llm_accel.PORT_OUT)
    assert n >= 8 * spec.hidden
    _, st = acc.op(llm_accel.OP_RESIDUAL_ADD, 0, 4, 0, 0, in_ptr=p_out,
                   aux_ptr=p_in, out_ptr=p_aux)
    assert st.code == 0
    got = acc.port_read(llm_accel.PORT_AUX, a.size).reshape(a.shape)
    assert np.array_equal(got, orc.residual(a, b))


def test_operators_leave_the_resident_path_intact():
    # Task 18, then operator commands (projection staging, ports, a KV
    # append at a position the resident path does not use), then Task 19:
    # the resident results still equal the oracle's.
    import llm_accel
    from helpers import oracle_from_synthetic, oracle_shape
    spec = workloads.CONFIG_A
    synth = workloads.SyntheticModel(spec, layers=1)
    om = oracle_from_synthetic(synth, oracle_shape(spec, layers=1))
    kv = om.new_kv()
    h0 = synth.hidden_rows(3)
    with llm_accel.Accelerator(accel_shape(spec, layers=1)) as acc:
        acc.load_model(synth)
        acc.upload(1, h0)
        _, want18, _ = om.task(kv, 18, 0, h0, 0)
        acc.task(18, 0, 3, 0, 1, 0)
        rng = np.random.default_rng(5)
        acc.run_feature(llm_accel.OP_FFN_DOWN, _ints(rng, (8, spec.inter), -900, 900))
        acc.run_feature(llm_accel.OP_Q_PROJECTION, _ints(rng, (8, spec.hidden), -900, 900))
        g, d, hk = _group(spec), spec.head_dim, spec.kv_heads
        acc.run_attention(llm_accel.OP_DECODE_SMOKE, _ints(rng, (hk, g, d), -500, 500),
                          (_ints(rng, (hk, d), -500, 500), _ints(rng, (hk, d), -500, 500)),
                          position=40)
        assert np.array_equal(acc.download(0, 3), want18)
        _, want19, _ = om.task(kv, 19, 0, want18, 0)
        acc.task(19, 0, 3, 0, 0, 1)
        assert np.array_equal(acc.download(1, 3), want19)
        k, v = acc.kv_read(0, 0, 0, 3)
        assert np.array_equal(k, kv[0][0, 0, :3]) and np.array_equal(v, kv[1][0, 0, :3])
