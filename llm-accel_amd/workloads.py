"""Seeded synthetic workloads of the benchmark configurations.

Values are drawn as real numbers and quantised into the reference's
formats (include/datatypes.hpp:8-15): weights Q4.12, embeddings / hidden
state and RMSNorm gammas Q8.8.  numpy's PCG64 generator, seeded, makes the
same arrays on every machine with this numpy; the oracle and the HIP path
both consume exactly these arrays.
"""
import numpy as np

SEED = 20260718


class ShapeSpec:
    def __init__(self, name, vocab, hidden, inter, layers, heads, kv_heads,
                 max_seq, w_range, emb_sigma, emb_clip_sigmas=4.0,
                 gamma_range=(0.5, 1.5)):
        self.name = name
        self.vocab = vocab
        self.hidden = hidden
        self.inter = inter
        self.layers = layers
        self.heads = heads
        self.kv_heads = kv_heads
        self.max_seq = max_seq
        self.w_range = w_range
        self.emb_sigma = emb_sigma
        self.emb_clip_sigmas = emb_clip_sigmas
        self.gamma_range = gamma_range

    @property
    def head_dim(self):
        return self.hidden // self.heads

    @property
    def kv_channels(self):
        return self.kv_heads * self.head_dim

    def proj_dims(self, proj):
        """(out_dim, in_dim) of projection id 0..6 (Q K V O gate up down)."""
        h, i, c = self.hidden, self.inter, self.kv_channels
        return [(h, h), (c, h), (c, h), (h, h), (i, h), (i, h), (h, i)][proj]

    def weight_bytes_per_layer(self):
        return 2 * sum(o * i for o, i in (self.proj_dims(p) for p in range(7)))


# BASELINE.json configs[0] (A) and configs[1..4] (B-shaped).
CONFIG_A = ShapeSpec("config-A", 1024, 256, 688, 1, 4, 2, 64,
                     w_range=0.25, emb_sigma=0.5)
CONFIG_B = ShapeSpec("qwen2.5-3b-layer", 151936, 2048, 11008, 1, 16, 2, 2048,
                     w_range=0.125, emb_sigma=0.3)


def with_layers(spec, layers, max_seq=None, vocab=None):
    import copy
    s = copy.copy(spec)
    s.layers = layers
    if max_seq is not None:
        s.max_seq = max_seq
    if vocab is not None:
        s.vocab = vocab
    return s


def q412(rng, n, real_range):
    lim = int(round(real_range * 4096))
    return rng.integers(-lim, lim + 1, size=n, dtype=np.int16)


def q88_normal(rng, n, sigma, clip_sigmas):
    v = rng.standard_normal(n) * sigma
    v = np.clip(v, -clip_sigmas * sigma, clip_sigmas * sigma)
    return np.clip(np.round(v * 256.0), -32768, 32767).astype(np.int16)


class SyntheticModel:
    """Row-major weights [layer][proj] and norms; embedding / LM head
    generated on request (the 151936-row table is 622 MB)."""

    def __init__(self, spec, seed=SEED, layers=None):
        self.spec = spec
        self.seed = seed
        n_layers = spec.layers if layers is None else layers
        rng = np.random.default_rng(seed)
        self._w = []
        for _ in range(n_layers):
            per = []
            for p in range(7):
                o, i = spec.proj_dims(p)
                per.append(q412(rng, o * i, spec.w_range).reshape(o, i))
            self._w.append(per)
        lo, hi = spec.gamma_range
        self._norms = rng.integers(int(round(lo * 256)), int(round(hi * 256)) + 1,
                                   size=(2 * n_layers + 1) * spec.hidden,
                                   dtype=np.int16).reshape(2 * n_layers + 1,
                                                           spec.hidden)

    def weight(self, layer, proj):
        return self._w[layer][proj]

    def plant_outliers(self, value=2048):
        """One weight of raw `value` (outside [-2048, 2047]: the 12-bit
        copies do not hold it) at row 0, column 0 of every matrix."""
        for per in self._w:
            for w in per:
                w[0, 0] = value

    def norms(self):
        return self._norms

    def embedding(self):
        rng = np.random.default_rng(self.seed + 1)
        return q88_normal(rng, self.spec.vocab * self.spec.hidden,
                          self.spec.emb_sigma,
                          self.spec.emb_clip_sigmas).reshape(self.spec.vocab,
                                                             self.spec.hidden)

    def lm_head(self):
        rng = np.random.default_rng(self.seed + 2)
        return q412(rng, self.spec.vocab * self.spec.hidden,
                    self.spec.w_range).reshape(self.spec.vocab,
                                               self.spec.hidden)

    def tokens(self, n, seed_offset=3):
        rng = np.random.default_rng(self.seed + seed_offset)
        return rng.integers(0, self.spec.vocab, size=n)

    def hidden_rows(self, n, seed_offset=4):
        rng = np.random.default_rng(self.seed + seed_offset)
        return q88_normal(rng, n * self.spec.hidden, self.spec.emb_sigma,
                          self.spec.emb_clip_sigmas).reshape(n, self.spec.hidden)

    def kv_rows(self, n, seed_offset=5):
        """Seeded Q8.8 K/V ~ N(0, 0.3) rows [n][head_dim] (config 4)."""
        rng = np.random.default_rng(self.seed + seed_offset)
        d = self.spec.head_dim
        k = q88_normal(rng, n * d, 0.3, 4.0).reshape(n, d)
        v = q88_normal(rng, n * d, 0.3, 4.0).reshape(n, d)
        return k, v
