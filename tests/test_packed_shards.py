"""The reference's packed weight format (16 shards of 64-byte words of
16x16 tiles, host/host_qwen_8x64.cpp:842-869 and projection_weight_raw
:899-935) in the oracle."""
import numpy as np
import pytest

from oracle import orc


def _slot(shape, layer, proj, out, inp):
    """projection_weight_raw's index computation (host:916-934), written in
    the accessor's forward direction (element -> shard, word, lane)."""
    def dims(p):
        H, I, C = shape.hidden_size, shape.intermediate_size, shape.kv_channels
        out_dim = I if p in (orc.PROJ_GATE, orc.PROJ_UP) else (
            C if p in (orc.PROJ_K, orc.PROJ_V) else H)
        in_dim = I if p == orc.PROJ_DOWN else H
        return out_dim, in_dim
    tiles = [(-(-dims(p)[0] // 16)) * (-(-dims(p)[1] // 16)) for p in range(7)]
    base = sum(tiles[:proj])
    in_tiles = -(-dims(proj)[1] // 16)
    g = layer * sum(tiles) + base + (out // 16) * in_tiles + inp // 16
    lane_in_tile = (out % 16) * 16 + inp % 16
    return (g & 1) * 8 + lane_in_tile // 32, g >> 1, lane_in_tile % 32


@pytest.mark.parametrize("profile", ["small", "medium"])
def test_load_shards_equals_reference_random_model(profile):
    s = orc.profile(profile)
    shards = orc.reference_random_shards(s, 20260718)
    a = orc.Model(s)
    a.init_reference_random(20260718)
    b = orc.Model(s, with_embedding=False)
    b.load_shards(shards)
    for layer in range(s.num_layers):
        for p in range(7):
            assert np.array_equal(a.weight(layer, p), b.weight(layer, p)), (layer, p)


def test_shard_slot_forward_accessor():
    s = orc.profile("medium")
    rng = np.random.default_rng(3)
    shards = [rng.integers(-2000, 2000, (orc.shard_words(s), 32),
                           dtype=np.int16) for _ in range(16)]
    m = orc.Model(s, with_embedding=False)
    m.load_shards(shards)
    for _ in range(400):
        layer = int(rng.integers(s.num_layers))
        p = int(rng.integers(7))
        w = m.weight(layer, p)
        o, i = int(rng.integers(w.shape[0])), int(rng.integers(w.shape[1]))
        sh, word, lane = _slot(s, layer, p, o, i)
        assert w[o, i] == shards[sh][word, lane], (layer, p, o, i)


def test_shards_too_small_rejected():
    s = orc.profile("small")
    words = orc.shard_words(s)
    m = orc.Model(s, with_embedding=False)
    with pytest.raises(ValueError):
        m.load_shards([np.zeros((words - 1, 32), np.int16)] * 16)
