"""Oracle primitives against what the mathematics fixes: closed forms,
exact rationals, invariants and special cases chosen so that a dropped
rounding term, a wrong shift or a transposed operand fails."""
import math
from decimal import ROUND_FLOOR, Decimal, getcontext
from fractions import Fraction

import numpy as np
import pytest

from oracle import orc

getcontext().prec = 60


@pytest.fixture(autouse=True)
def _reference_tables():
    orc.set_exp_policy(orc.EXP_HLS, orc.EXP_HLS)
    yield


def _floor_exp(x_raw, frac_bits):
    v = (Decimal(x_raw) / 256).exp() * (Decimal(2) ** frac_bits)
    return int(v.to_integral_value(rounding=ROUND_FLOOR))


def test_q2_14_table_is_floor_of_exact_exp():
    # hls::exp<18,4> (host:588-596), pinned by KAT-1's post-attention
    # fingerprint (tests/test_oracle_kat.py).
    _, q14 = orc.exp_tables()
    for x in range(-2048, 1):
        assert q14[x + 2048] == _floor_exp(x, 14), x
    assert q14[2048] == 16384  # e^0


def _hls_exp_data():
    import json
    import os
    here = os.path.dirname(os.path.abspath(__file__))
    return json.load(open(os.path.join(here, "golden", "hls_exp_q8_8.json")))


def test_q8_8_table_equals_recovered_hls_exp():
    """The oracle's hls::exp<16,8> restatement equals the table that
    tests/golden/exp_q8_8_search.py recovered (with exact decimal
    arithmetic) and confirmed against KAT-1/2/3, over the whole clamped
    input range [-8, 8]."""
    d = _hls_exp_data()
    full = np.array([orc.lib.orc_exp_q8_8(x) for x in range(-2048, 2049)])
    assert list(full[2048::-1]) == d["neg_table"]
    assert list(full[2048:]) == d["pos_table"]


def test_q8_8_table_shape_of_the_hls_construction():
    """What the construction fixes independently of the fixtures: e^0 is
    exactly 1.0; every entry is within one unit of floor(e^x * 256);
    entries at the half-integer grid points (lsb and msb_2 fields zero) are
    E1 = e^x rounded at 14 bits, then truncated to 8; and the recovered
    E1 / E2 constants are e^x and e^x - 1 rounded at 14 and 26 bits."""
    d = _hls_exp_data()
    neg = d["neg_table"]
    assert neg[0] == 256
    for k in range(2049):
        assert abs(neg[k] - _floor_exp(-k, 8)) <= 1, k
    for v, e1 in d["E1"].items():
        v = int(v)
        exact = (Decimal(v) / 256).exp() * (1 << 14)
        assert e1 == int((exact + Decimal("0.5")).to_integral_value(rounding=ROUND_FLOOR))
        if v <= 0:
            assert neg[-v] == e1 >> 6, v
    for v, e2 in d["E2m1"].items():
        exact = ((Decimal(int(v)) / 256).exp() - 1) * (1 << 26)
        assert e2 == int((exact + Decimal("0.5")).to_integral_value(rounding=ROUND_FLOOR))
    # 13 entries differ from floor(e^x * 256) in [-8, 0]
    assert sum(neg[k] != _floor_exp(-k, 8) for k in range(2049)) == 13


def test_product_exp_tables_equal_oracle():
    import llm_accel
    a, b = llm_accel.exp_tables()
    q8, q14 = orc.exp_tables()
    assert np.array_equal(a, q8) and np.array_equal(b, q14)


# ---- reciprocal / rsqrt -------------------------------------------------
def test_recip_powers_of_two_and_zero():
    # Newton from a power-of-two seed is exact on powers of two.
    for k in range(-3, 7):
        x = int(256 * 2.0 ** k)
        assert orc.lib.orc_recip(x) == int(round(256 / 2.0 ** k)), k
    # recip(0): safe = 0, est 16 -> 32 -> 64 -> 128 (sat 127.996) -> clamp 64
    assert orc.lib.orc_recip(0) == 16384
    assert orc.lib.orc_recip(-5) == 16384


def test_recip_follows_newton_closed_form():
    # Three exact Newton steps from seed s give (1 - (1 - x*s)^8) / x; the
    # Q8.8 rounding of each step adds at most a few LSB.
    for x in range(256, 16384, 7):  # [1, 64)
        xf = x / 256
        s = 2.0 ** -math.floor(math.log2(xf))
        want = (1 - (1 - xf * s) ** 8) / xf * 256
        assert abs(orc.lib.orc_recip(x) - want) <= 4.0, x


def _q(x, F, W):
    """ap_fixed assignment: AP_RND (floor(x*2^F + 1/2)) then AP_SAT."""
    r = math.floor(x * 2 ** F + Fraction(1, 2))
    lo, hi = -(1 << (W - 1)), (1 << (W - 1)) - 1
    return Fraction(max(lo, min(hi, r)), 2 ** F)


def _recip_exact_chain(x_raw):
    """golden_recip as exact rationals, quantising on every assignment."""
    x = Fraction(x_raw, 256)
    safe = x if x >= _q(Fraction(1, 4096), 8, 16) else _q(Fraction(1, 4096), 8, 16)
    est = Fraction(16)
    for th, e in ((64, Fraction(1, 64)), (32, Fraction(1, 32)), (16, Fraction(1, 16)),
                  (8, Fraction(1, 8)), (4, Fraction(1, 4)), (2, Fraction(1, 2)),
                  (1, Fraction(1)), (Fraction(1, 2), Fraction(2)),
                  (Fraction(1, 4), Fraction(4)), (Fraction(1, 8), Fraction(8))):
        if safe >= th:
            est = e
            break
    for _ in range(3):
        est = _q(est * (2 - safe * est), 8, 16)
    return int(min(max(est, Fraction(0)), Fraction(64)) * 256)


def test_recip_matches_exact_rational_chain_exhaustively():
    for x in range(-32768, 32768, 1):
        assert orc.lib.orc_recip(x) == _recip_exact_chain(x), x


def test_recip_saturated_input_collapses_to_zero():
    # fm(H) for H >= 128 saturates to 127.996; the first Newton step then
    # underflows to 0 (degenerate RMSNorm, reference host:3179-3185).
    assert orc.lib.orc_recip(32767) == 0


def test_rsqrt_closed_forms():
    assert orc.lib.orc_rsqrt(1 << 16) == 256      # 1/sqrt(1)
    assert orc.lib.orc_rsqrt(4 << 16) == 128      # 1/sqrt(4)
    assert orc.lib.orc_rsqrt(16 << 16) == 64
    # Degenerate RMSNorm chain on the 2^-12 floor: seed 8 -> 11.9375 ->
    # 17.69921875 -> 25.87109375 (= 6623 / 256).
    assert orc.lib.orc_rsqrt(0) == 6623


def _rsqrt_exact_chain(v_raw):
    """golden_rsqrt as exact rationals with ap_fixed quantisation on every
    assignment (AP_RND = floor(x*2^F + 1/2), AP_SAT)."""
    def q(x, F, W):
        r = math.floor(x * 2 ** F + Fraction(1, 2))
        lo, hi = -(1 << (W - 1)), (1 << (W - 1)) - 1
        return Fraction(max(lo, min(hi, r)), 2 ** F)
    safe = max(Fraction(v_raw, 1 << 16), Fraction(1, 4096))
    seeds = [(64, 0.125), (16, 0.25), (4, 0.5), (1, 1), (0.25, 2), (0.0625, 4)]
    est = Fraction(8)
    for th, e in seeds:
        if safe >= Fraction(th):
            est = Fraction(e)
            break
    for _ in range(3):
        sq = q(est * est, 16, 32)
        refine = q(Fraction(3, 2) - Fraction(1, 2) * safe * sq, 16, 32)
        est = q(est * refine, 8, 16)
    est = min(max(est, Fraction(0)), Fraction(32))
    return int(est * 256)


def test_rsqrt_matches_exact_rational_chain():
    rng = np.random.default_rng(7)
    vals = list(rng.integers(0, 1 << 31, 300)) + [0, 15, 16, 17, 4095, 4096,
                                                   1 << 16, (1 << 31) - 1]
    for v in vals:
        assert orc.lib.orc_rsqrt(int(v)) == _rsqrt_exact_chain(int(v)), v


# ---- RMSNorm -------------------------------------------------------------
@pytest.mark.parametrize("cols", [128, 256, 2048])
def test_rmsnorm_degenerate_gain_for_wide_rows(cols):
    rng = np.random.default_rng(cols)
    x = rng.integers(-3000, 3000, (4, cols), dtype=np.int16)
    g = rng.integers(128, 384, cols, dtype=np.int16)
    y = orc.rmsnorm(x, g)
    prod = x.astype(np.int64) * 6623 * g.astype(np.int64)
    want = np.clip((prod + (1 << 15)) >> 16, -32768, 32767)
    assert np.array_equal(y, want)


def test_rmsnorm_normal_regime_small_rows():
    # H = 64 (reference 'small' profile): inv_elems = 1/64 is exact, so the
    # output tracks x * gamma / rms within the Q8.8 Newton precision.
    rng = np.random.default_rng(3)
    x = rng.integers(-512, 512, (6, 64), dtype=np.int16)
    g = np.full(64, 256, np.int16)
    y = orc.rmsnorm(x, g).astype(float) / 256
    xf = x.astype(float) / 256
    ref = xf / np.sqrt((xf ** 2).mean(axis=1, keepdims=True))
    assert np.max(np.abs(y - ref)) < 0.08


# ---- projection ------------------------------------------------------------
def test_projection_double_rounding_is_not_single_rounding():
    # acc = 2047 raw Q28.20: Q16.16 rounds to 128 (0.5 LSB of Q8.8), which
    # then rounds up to 1; a single rounding would give 0.
    x = np.array([[1]], np.int16)
    w = np.array([[2047]], np.int16)
    assert orc.projection(x, w)[0, 0] == 1
    w = np.array([[2039]], np.int16)
    assert orc.projection(x, w)[0, 0] == 0


def test_projection_matches_exact_integer_product():
    rng = np.random.default_rng(11)
    x = rng.integers(-32768, 32768, (5, 300), dtype=np.int16)
    w = rng.integers(-32768, 32768, (37, 300), dtype=np.int16)
    acc = x.astype(object) @ w.astype(object).T  # exact Python ints
    def q(v, s):
        return (v + (1 << (s - 1))) >> s
    want = np.vectorize(lambda a: max(-32768, min(32767, q(max(-(1 << 31), min((1 << 31) - 1, q(a, 4))), 8))))(acc)
    assert np.array_equal(orc.projection(x, w), want.astype(np.int16))


def test_projection_saturates():
    x = np.full((1, 64), 32767, np.int16)
    w = np.full((2, 64), 32767, np.int16)
    w[1] = -32768
    y = orc.projection(x, w)
    assert y[0, 0] == 32767 and y[0, 1] == -32768


# ---- attention ----------------------------------------------------------------
def test_qk_score_closed_form():
    # q = 1.0 at one lane, k = 1.0 there: dot 1.0; scale fm(1/sqrt(128)) is
    # raw 23 (0.08984375); the score is raw 23.
    q = np.zeros((1, 128), np.int16)
    k = np.zeros((1, 128), np.int16)
    q[0, 5] = 256
    k[0, 5] = 256
    assert orc.qk_scores(q, k)[0, 0] == 23
    # d = 64: scale 0.125 -> raw 32.
    assert orc.qk_scores(q[:, :64], k[:, :64])[0, 0] == 32
    # K saturates to +-8 in Q4.12: k = 16.0 acts as 7.99976
    k[0, 5] = 4096
    q[0, 5] = 256 * 4
    # 4 * 7.999755859375 = 31.9990234375 -> *0.08984375 -> 2.8749 -> raw 736
    assert orc.qk_scores(q, k)[0, 0] == 736


def test_single_position_attention_is_saturated_v():
    # softmax over one entry is exactly 1.0 (Q2.14 16384); PV x 64 / 64
    # returns V converted to Q4.12, i.e. clamped to [-8, 8].
    rng = np.random.default_rng(5)
    for d in (64, 128):
        q = rng.integers(-4000, 4000, (8, d), dtype=np.int16)
        k = rng.integers(-4000, 4000, (1, d), dtype=np.int16)
        v = rng.integers(-6000, 6000, (1, d), dtype=np.int16)
        out = orc.attention(q, k, v)
        want = np.clip(v, -2048, 2048)
        assert np.array_equal(out, np.repeat(want, 8, axis=0))


@pytest.mark.parametrize("semantics", [orc.SEM_RAW_PAYLOAD, orc.SEM_LEGACY_Q8_8])
@pytest.mark.parametrize("n", [1, 5, 64, 65, 200])
def test_uniform_scores_give_rounded_mean(n, semantics):
    """q = 0 makes every score 0, every probability 1.0 and every rescale
    factor 1.0 after the first tile, so the output is a closed form in the
    per-tile sums of V: floor(sum_t sat16(sum_tile v) * inv / 256 + 1/2)
    with inv = floor(256 / n + 1/2).  Both probability formats (Q2.14 with
    the PV result scaled by 1/64, Q8.8 unscaled) reach the same form."""
    rng = np.random.default_rng(n)
    d = 64
    q = np.zeros((2, d), np.int16)
    k = rng.integers(-3000, 3000, (n, d), dtype=np.int16)
    v = rng.integers(-60, 60, (n, d), dtype=np.int16)
    out = orc.attention(q, k, v, semantics)
    inv = math.floor(Fraction(256, n) + Fraction(1, 2))
    tiles = [v[t:t + 64].astype(np.int64).sum(axis=0) for t in range(0, n, 64)]
    acc = sum(np.clip(t, -32768, 32767) for t in tiles) * 256
    want = np.floor((acc * inv) / 65536 + 0.5).astype(np.int64)
    assert np.array_equal(out[0], want) and np.array_equal(out[1], want)


def test_legacy_single_position_is_saturated_v():
    # Q8.8 probabilities: exp(0) = 1.0 is raw 256, the sum 1.0, and the
    # unscaled PV of 256 x Q4.12(v) returns v clamped to [-8, 8].
    rng = np.random.default_rng(6)
    q = rng.integers(-4000, 4000, (8, 128), dtype=np.int16)
    k = rng.integers(-4000, 4000, (1, 128), dtype=np.int16)
    v = rng.integers(-6000, 6000, (1, 128), dtype=np.int16)
    out = orc.attention(q, k, v, orc.SEM_LEGACY_Q8_8)
    assert np.array_equal(out, np.repeat(np.clip(v, -2048, 2048), 8, axis=0))


def test_legacy_one_tile_composes_scores_exp8_pv_and_inverse():
    """Within one tile the Q8.8 recurrence starts from sum 0 and acc 0, so
    the output is fm(256 * PV(p, v) * inv(sum p)) with p = exp8(s - max):
    checks that the legacy path uses the Q8.8 table and no 1/64 scale,
    from the separately pinned scores, table, PV and inverse."""
    rng = np.random.default_rng(17)
    n, d = 37, 64
    q = rng.integers(-900, 900, (4, d), dtype=np.int16)
    k = rng.integers(-900, 900, (n, d), dtype=np.int16)
    v = rng.integers(-700, 700, (n, d), dtype=np.int16)
    s = orc.qk_scores(q, k).astype(np.int64)
    p = np.array([[orc.lib.orc_exp_q8_8(int(np.clip(x - row.max(), -32768, 32767)))
                   for x in row] for row in s], np.int16)
    pv = orc.attention_pv(p, v).astype(np.int64)
    inv = np.array([orc.lib.orc_inv_sum(int(r.astype(np.int64).sum()) * 256) for r in p],
                   np.int64)
    want = np.clip(np.floor((pv * 256 * inv[:, None]) / 65536 + 0.5), -32768, 32767)
    assert np.array_equal(orc.attention(q, k, v, orc.SEM_LEGACY_Q8_8), want)
    # the production format differs (Q2.14 probabilities)
    assert not np.array_equal(orc.attention(q, k, v), want)


# ---- ATTN_PV and SOFTMAX operators ----------------------------------------------
def test_attention_pv_one_hot_selects_the_saturated_v_row():
    # p = 1.0 (raw 256) at position j: 256 x Q4.12(v) / 256 = v clamped to
    # [-8, 8]; columns past n are ignored.
    rng = np.random.default_rng(3)
    n, d = 13, 128
    v = rng.integers(-3000, 3000, (n, d), dtype=np.int16)
    p = np.zeros((8, 64), np.int16)
    p[:, n:] = 32767
    sel = rng.integers(0, n, 8)
    p[np.arange(8), sel] = 256
    out = orc.attention_pv(p, v)
    assert np.array_equal(out, np.clip(v[sel], -2048, 2048))


def test_attention_pv_is_a_sum_over_positions():
    # Two selected positions add (small values: no rounding, no saturation);
    # a transposed operand or a dropped bank fails this.
    rng = np.random.default_rng(4)
    n, d = 64, 64
    v = rng.integers(-500, 500, (n, d), dtype=np.int16)
    p = np.zeros((3, 64), np.int16)
    pairs = [(0, 5), (6, 63), (33, 34)]
    for r, (a, b) in enumerate(pairs):
        p[r, a] = p[r, b] = 256
    out = orc.attention_pv(p, v)
    for r, (a, b) in enumerate(pairs):
        assert np.array_equal(out[r], v[a].astype(np.int32) + v[b])
    # p = 0.5 (raw 128): half of the row, rounded half up
    p2 = np.zeros((1, 64), np.int16)
    p2[0, 9] = 128
    assert np.array_equal(orc.attention_pv(p2, v)[0],
                          np.floor(v[9] / 2 + 0.5).astype(np.int64))


@pytest.mark.parametrize("n", [1, 2, 4, 13, 64])
def test_softmax_of_equal_values_is_the_reciprocal(n):
    # every exp is 1.0 (raw 256), the sum is n, the result recip(n) (the
    # pinned Newton reciprocal); columns past n are ignored
    x = np.full((2, 64), -700, np.int16)
    x[:, n:] = 30000
    out = orc.softmax_rows(x, n)
    want = orc.lib.orc_recip(256 * n) if 256 * n <= 32767 else orc.lib.orc_recip(32767)
    assert out.shape == (2, n) and np.all(out == want)
    if n in (1, 2, 4):
        assert want == 256 // n


def test_softmax_dominant_entry_and_normalisation():
    rng = np.random.default_rng(8)
    # one entry 8 or more above the rest: exp(-8) is raw 0, the row is one-hot
    x = rng.integers(-3000, -2000, (4, 64)).astype(np.int16)
    x[np.arange(4), [0, 7, 31, 63]] = 0
    out = orc.softmax_rows(x, 64)
    assert np.array_equal(out, np.eye(64, dtype=np.int16)[[0, 7, 31, 63]] * 256)
    # general rows: fm(e * recip(sum e)) with e from the pinned Q8.8 table
    # and the pinned Newton reciprocal (three steps from a power-of-two
    # seed: not the exact 1 / sum, so the rows need not sum to 1.0)
    x = rng.integers(-1500, 1500, (6, 64)).astype(np.int16)
    for n in (5, 40, 64):
        out = orc.softmax_rows(x, n)
        for r in range(6):
            e = np.array([orc.lib.orc_exp_q8_8(int(np.clip(int(a) - int(x[r, :n].max()),
                                                            -32768, 32767)))
                          for a in x[r, :n]], np.int64)
            inv = orc.lib.orc_recip(int(min(e.sum(), 32767)))
            assert np.array_equal(out[r], np.floor(e * inv / 256 + 0.5).astype(np.int64))
            assert out[r].argmax() == x[r, :n].argmax()


def test_attention_tiles_anchor_at_zero_and_prefix_invariance():
    # Appending positions never changes earlier rows' results (causality
    # of the incremental cache) and tiles are anchored at position 0: the
    # result for n positions only depends on the first n K/V rows.
    rng = np.random.default_rng(9)
    q = rng.integers(-800, 800, (4, 64), dtype=np.int16)
    k = rng.integers(-800, 800, (150, 64), dtype=np.int16)
    v = rng.integers(-800, 800, (150, 64), dtype=np.int16)
    a = orc.attention(q, k[:100], v[:100])
    k2 = k.copy()
    k2[100:] = 12345
    b = orc.attention(q, k2[:100], v[:100])
    assert np.array_equal(a, b)


# ---- RoPE ---------------------------------------------------------------------
def _half_away(x):
    return int(math.copysign(math.floor(abs(x) + 0.5), x))


def test_rope_table_matches_libm_rounded_half_away():
    t = orc.rope_table(40, 128)
    for p in (0, 1, 7, 39):
        for i in range(64):
            ang = p * (1.0 / math.pow(1e6, (2 * i) / 128))
            assert t[p, i] == _half_away(math.cos(ang) * 256)
            assert t[p, 64 + i] == _half_away(math.sin(ang) * 256)


def test_rope_position_zero_is_identity():
    t = orc.rope_table(1, 128)
    rng = np.random.default_rng(1)
    x = rng.integers(-32768, 32768, 4 * 128, dtype=np.int16)
    assert np.array_equal(orc.rope_apply(x, 4, 128, t[0]), x)


def test_rope_quarter_turn_swaps_halves():
    # cos = 0, sin = 1 maps (x0, x1) -> (-x1, x0).
    row = np.zeros(8, np.int16)
    row[4:] = 256
    x = np.array([1, 2, 3, 4, 10, 20, 30, 40], np.int16)
    assert list(orc.rope_apply(x, 1, 8, row)) == [-10, -20, -30, -40, 1, 2, 3, 4]


# ---- SiLU -----------------------------------------------------------------------
def test_silu_closed_points():
    assert orc.lib.orc_silu(0) == 0
    # large positive: e^-x underflows the table to 0, recip(1) = 1 -> x
    assert orc.lib.orc_silu(2048) == 2048
    # large negative: e^-8 floors to 0 in Q8.8 -> 0
    assert orc.lib.orc_silu(-4096) == 0


def test_silu_tracks_float_silu():
    xs = np.arange(-2048, 2048, 3)
    got = np.array([orc.lib.orc_silu(int(x)) for x in xs]) / 256
    xf = xs / 256
    ref = xf / (1 + np.exp(-xf))
    assert np.max(np.abs(got - ref)) < 0.05


# ---- host helpers ---------------------------------------------------------
def test_fnv1a_over_uint16():
    assert orc.checksum(np.zeros(0, np.int16)) == 1469598103934665603
    c = 1469598103934665603
    for v in (1, -1, 300):
        c ^= v & 0xFFFF
        c = (c * 1099511628211) % (1 << 64)
    assert orc.checksum(np.array([1, -1, 300], np.int16)) == c


def test_lm_head_argmax_first_index_on_ties():
    table = np.array([[1, 2], [3, 0], [1, 2], [0, 0]], np.int16)
    h = np.array([2, 1], np.int16)  # scores 4, 6, 4, 0
    assert orc.lm_head_argmax(table, h) == 1
    table[1] = [1, 2]  # scores 4, 4, 4, 0 -> first
    assert orc.lm_head_argmax(table, h) == 0
    rng = np.random.default_rng(2)
    t = rng.integers(-32768, 32768, (500, 64), dtype=np.int16)
    hh = rng.integers(-32768, 32768, 64, dtype=np.int16)
    assert orc.lm_head_argmax(t, hh) == int(np.argmax(t.astype(np.int64) @ hh.astype(np.int64)))


# ---- composition invariants ------------------------------------------------
def test_incremental_decode_equals_full_prefix_recompute():
    """The reference validates decode by a full-prefix recompute
    (host:9153-9172); with a causal cache both give identical rows."""
    s = orc.shape(64, 256, 688, 1, 4, 2, 64)
    m = orc.Model(s, 1, False)
    rng = np.random.default_rng(4)
    for p in range(7):
        w = m.weight(0, p)
        w[:] = rng.integers(-1024, 1025, w.shape, dtype=np.int16)
    m.norms()[:] = rng.integers(128, 385, m.norms().shape, dtype=np.int16)
    h = rng.integers(-400, 400, (11, 256), dtype=np.int16)
    kv = m.new_kv()
    outs = []
    for pos, rows in ((0, 8), (8, 2), (10, 1)):
        _, x, _ = m.task(kv, 18, 0, h[pos:pos + rows], pos)
        _, x, _ = m.task(kv, 19, 0, x, pos)
        outs.append(x)
    inc = np.concatenate(outs)
    _, full = m.prefill_sequence(h, 0)
    assert np.array_equal(inc, full)


def test_status_validation_order():
    s = orc.shape(64, 256, 688, 1, 4, 2, 64)
    m = orc.Model(s, 1, False)
    kv = m.new_kv()
    h = np.zeros((8, 256), np.int16)
    expect = {
        (18, 0, 9, 0): (0, 2), (18, 0, 0, 0): (18, 2), (21, 0, 1, 0): (21, 1),
        (5, 0, 1, 0): (5, 1), (5, 3, 1, 0): (5, 5), (18, 1, 1, 0): (18, 5),
        (18, 0, 1, 64): (18, 4), (18, 0, 4, 61): (18, 4), (20, 0, 0, 0): (20, 2),
        (0, 0, 3, 0): (0, 0), (17, 0, 2, 0): (17, 1), (16, 0, 8, 56): (16, 0),
    }
    for (op, layer, rows, pos), (sop, code) in expect.items():
        c, _, st = m.task(kv, op, layer, h, pos, token_count=rows)
        assert (st.op, st.code, c, st.last_task) == (sop, code, code, 1)
        assert st.token_count == rows


def test_byte_split_dot_product_identity():
    """The matrix-core projection computes sum w*x from byte planes:
    w = 256a + b + 128, x = 256c + d + 128 with a = w >> 8,
    b = (w & 255) - 128 (c, d likewise), all in [-128, 127], and
    sum wx = 65536 sum ac + 256 (sum ad + sum bc) + sum bd + 32768 sum a
             + 128 sum b + 32768 sum c + 128 sum d + 16384 K.
    Checked on random and extreme int16 vectors against the direct sum."""
    rng = np.random.default_rng(11)
    extremes = np.array([-32768, -32767, -256, -129, -128, -1, 0, 1, 127,
                         128, 255, 256, 32512, 32639, 32640, 32767], np.int64)
    for trial in range(200):
        k = int(rng.integers(1, 300))
        if trial % 3 == 0:
            w = rng.choice(extremes, k)
            x = rng.choice(extremes, k)
        else:
            w = rng.integers(-32768, 32768, k)
            x = rng.integers(-32768, 32768, k)
        a, b = w >> 8, (w & 255) - 128
        c, d = x >> 8, (x & 255) - 128
        for v in (a, b, c, d):
            assert v.min() >= -128 and v.max() <= 127
        got = (65536 * (a * c).sum() + 256 * ((a * d).sum() + (b * c).sum())
               + (b * d).sum() + 32768 * a.sum() + 128 * b.sum()
               + 32768 * c.sum() + 128 * d.sum() + 16384 * k)
        assert got == int((w * x).sum())
        # bounds the kernel relies on: each plane product <= 2^14 in size
        assert np.abs(a * c).max() <= 1 << 14
