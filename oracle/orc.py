"""ctypes binding of the CPU oracle (oracle/liborc.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg, as the checker.  The product path never
imports this module.
"""
import ctypes
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liborc.so")

EXP_FLOOR, EXP_ROUND, EXP_HLS = 0, 1, 2
UID_DIVREJ, UID_LEMIRE = 0, 1
SEM_RAW_PAYLOAD, SEM_DIRECT, SEM_LEGACY_Q8_8 = 0, 1, 2
PROJ_Q, PROJ_K, PROJ_V, PROJ_O, PROJ_GATE, PROJ_UP, PROJ_DOWN = range(7)

_i16p = ctypes.POINTER(ctypes.c_int16)
_i32p = ctypes.POINTER(ctypes.c_int32)
_u32 = ctypes.c_uint32


class Shape(ctypes.Structure):
    _fields_ = [(n, ctypes.c_uint32) for n in (
        "vocab_size", "hidden_size", "intermediate_size", "num_layers",
        "num_heads", "num_kv_heads", "max_seq_len")]

    @property
    def head_dim(self):
        return self.hidden_size // self.num_heads

    @property
    def kv_channels(self):
        return self.num_kv_heads * self.head_dim

    @property
    def group(self):
        return self.num_heads // self.num_kv_heads


class Status(ctypes.Structure):
    _fields_ = [(n, ctypes.c_uint32) for n in (
        "op", "code", "token_count", "output_waves", "mm_tasks",
        "vector_tasks", "completed_packets", "last_task")]

    def as_tuple(self):
        return tuple(getattr(self, n) for n, _ in self._fields_)


def _load():
    if not os.path.exists(_LIB_PATH):
        raise RuntimeError(
            "oracle library missing: build it with `make -C oracle`")
    lib = ctypes.CDLL(_LIB_PATH)
    sig = {
        "orc_set_exp_policy": (None, [ctypes.c_int, ctypes.c_int]),
        "orc_exp_q8_8": (ctypes.c_int16, [ctypes.c_int16]),
        "orc_attn_prob": (ctypes.c_int16, [ctypes.c_int16]),
        "orc_get_exp_tables": (None, [_i16p, _i16p]),
        "orc_set_exp_tables": (None, [_i16p, _i16p]),
        "orc_recip": (ctypes.c_int16, [ctypes.c_int16]),
        "orc_rsqrt": (ctypes.c_int16, [ctypes.c_int32]),
        "orc_silu": (ctypes.c_int16, [ctypes.c_int16]),
        "orc_quantize_fix16": (ctypes.c_int16, [ctypes.c_double]),
        "orc_inv_sum": (ctypes.c_int16, [ctypes.c_int32]),
        "orc_fm_wt_term": (ctypes.c_int32, [ctypes.c_int16, ctypes.c_int16]),
        "orc_projection": (None, [_i16p, _u32, _u32, _i16p, _u32, _i16p]),
        "orc_residual": (None, [_i16p, _i16p, ctypes.c_size_t, _i16p]),
        "orc_rmsnorm": (None, [_i16p, _u32, _u32, _i16p, _i16p]),
        "orc_silu_mul": (None, [_i16p, _i16p, ctypes.c_size_t, _i16p]),
        "orc_rope_table": (None, [_u32, _u32, ctypes.c_double, _i16p]),
        "orc_rope_apply": (None, [_i16p, _u32, _u32, _i16p]),
        "orc_attention": (None, [_i16p, _u32, _u32, _i16p, _i16p, _u32,
                                 ctypes.c_int, _i16p]),
        "orc_qk_scores": (None, [_i16p, _u32, _u32, _i16p, _u32, _i16p]),
        "orc_attention_pv": (None, [_i16p, _u32, _u32, _i16p, _u32, _u32,
                                    _i16p]),
        "orc_softmax_rows": (None, [_i16p, _u32, _u32, _u32, _i16p]),
        "orc_model_create": (ctypes.c_void_p,
                             [ctypes.POINTER(Shape), _u32, ctypes.c_int]),
        "orc_model_destroy": (None, [ctypes.c_void_p]),
        "orc_model_weight": (_i16p, [ctypes.c_void_p, _u32, _u32]),
        "orc_model_norms": (_i16p, [ctypes.c_void_p]),
        "orc_model_embedding": (_i16p, [ctypes.c_void_p]),
        "orc_model_init_reference_random": (None, [ctypes.c_void_p, _u32,
                                                   ctypes.c_int]),
        "orc_make_random_tensor": (None, [_u32, _u32, _u32, ctypes.c_int32,
                                          ctypes.c_int32, ctypes.c_int,
                                          _i16p]),
        "orc_lm_head_argmax": (_u32, [_i16p, _u32, _u32, _i16p]),
        "orc_checksum": (ctypes.c_uint64, [_i16p, ctypes.c_size_t]),
        "orc_mt19937_nth": (ctypes.c_uint32, [_u32, ctypes.c_uint64]),
        "orc_uniform_ints": (None, [_u32, ctypes.c_int32, ctypes.c_int32,
                                    ctypes.c_int, ctypes.c_size_t, _i32p]),
        "orc_set_threads": (None, [ctypes.c_int]),
        "orc_reference_random_shards": (ctypes.c_int, [
            ctypes.c_void_p, _u32, ctypes.c_int, ctypes.c_uint64,
            ctypes.POINTER(_i16p)]),
        "orc_shard_words": (ctypes.c_uint64, [ctypes.c_void_p]),
        "orc_model_load_shards": (ctypes.c_int, [ctypes.c_void_p,
                                                 ctypes.POINTER(_i16p),
                                                 ctypes.c_uint64]),
        "orc_task": (ctypes.c_int, [ctypes.c_void_p, _i16p, _i16p, _u32,
                                    _u32, _u32, _u32, _i16p, _i16p,
                                    ctypes.c_int, ctypes.POINTER(Status)]),
        "orc_prefill_layer_sequence": (None, [ctypes.c_void_p, _i16p, _u32,
                                              _u32, ctypes.c_int, _i16p,
                                              _i16p]),
    }
    for name, (res, args) in sig.items():
        f = getattr(lib, name)
        f.restype = res
        f.argtypes = args
    return lib


lib = _load()


def p16(a):
    assert a.dtype == np.int16 and a.flags["C_CONTIGUOUS"]
    return a.ctypes.data_as(_i16p)


def set_exp_policy(q8_8=EXP_HLS, q2_14=EXP_HLS):
    lib.orc_set_exp_policy(q8_8, q2_14)


def set_exp_tables(q8_8=None, q2_14=None):
    """Install explicit tables (q8_8: 4097 entries for x raw -2048..2048,
    q2_14: 2049 entries for x raw -2048..0)."""
    a = None if q8_8 is None else np.ascontiguousarray(q8_8, np.int16)
    b = None if q2_14 is None else np.ascontiguousarray(q2_14, np.int16)
    if a is not None:
        assert a.shape == (4097,)
    if b is not None:
        assert b.shape == (2049,)
    lib.orc_set_exp_tables(None if a is None else p16(a),
                           None if b is None else p16(b))


def exp_tables():
    a = np.zeros(2049, np.int16)
    b = np.zeros(2049, np.int16)
    lib.orc_get_exp_tables(p16(a), p16(b))
    return a, b


def projection(x, w):
    x = np.ascontiguousarray(x, np.int16)
    w = np.ascontiguousarray(w, np.int16)
    rows, k = x.shape
    n = w.shape[0]
    assert w.shape[1] == k
    y = np.zeros((rows, n), np.int16)
    lib.orc_projection(p16(x), rows, k, p16(w), n, p16(y))
    return y


def rmsnorm(x, gamma):
    x = np.ascontiguousarray(x, np.int16)
    gamma = np.ascontiguousarray(gamma, np.int16)
    y = np.zeros_like(x)
    lib.orc_rmsnorm(p16(x), x.shape[0], x.shape[1], p16(gamma), p16(y))
    return y


def residual(a, b):
    a = np.ascontiguousarray(a, np.int16)
    b = np.ascontiguousarray(b, np.int16)
    y = np.zeros_like(a)
    lib.orc_residual(p16(a), p16(b), a.size, p16(y))
    return y


def silu_mul(g, u):
    g = np.ascontiguousarray(g, np.int16)
    u = np.ascontiguousarray(u, np.int16)
    y = np.zeros_like(g)
    lib.orc_silu_mul(p16(g), p16(u), g.size, p16(y))
    return y


def rope_table(max_seq, head_dim, theta=1e6):
    t = np.zeros((max_seq, head_dim), np.int16)
    lib.orc_rope_table(max_seq, head_dim, theta, p16(t))
    return t


def rope_apply(vec, heads, head_dim, row):
    vec = np.ascontiguousarray(vec, np.int16).copy()
    row = np.ascontiguousarray(row, np.int16)
    lib.orc_rope_apply(p16(vec), heads, head_dim, p16(row))
    return vec


def attention(q, k, v, semantics=SEM_RAW_PAYLOAD):
    q = np.ascontiguousarray(q, np.int16)
    k = np.ascontiguousarray(k, np.int16)
    v = np.ascontiguousarray(v, np.int16)
    g, d = q.shape
    out = np.zeros((g, d), np.int16)
    lib.orc_attention(p16(q), g, d, p16(k), p16(v), k.shape[0], semantics,
                      p16(out))
    return out


def attention_pv(p, v):
    """ATTN_PV: p [G][>= n] Q8.8 probabilities, v [n][d]."""
    p = np.ascontiguousarray(p, np.int16)
    v = np.ascontiguousarray(v, np.int16)
    n, d = v.shape
    out = np.zeros((p.shape[0], d), np.int16)
    lib.orc_attention_pv(p16(p), p.shape[0], p.shape[1], p16(v), n, d, p16(out))
    return out


def softmax_rows(x, n):
    """SOFTMAX over the first n elements of each row of x."""
    x = np.ascontiguousarray(x, np.int16)
    out = np.zeros((x.shape[0], n), np.int16)
    lib.orc_softmax_rows(p16(x), x.shape[0], x.shape[1], n, p16(out))
    return out


def qk_scores(q, k):
    q = np.ascontiguousarray(q, np.int16)
    k = np.ascontiguousarray(k, np.int16)
    out = np.zeros((q.shape[0], k.shape[0]), np.int16)
    lib.orc_qk_scores(p16(q), q.shape[0], q.shape[1], p16(k), k.shape[0],
                      p16(out))
    return out


def make_random_tensor(rows, cols, seed, lo=-128, hi=128, uid=UID_DIVREJ):
    out = np.zeros((rows, cols), np.int16)
    lib.orc_make_random_tensor(rows, cols, seed, lo, hi, uid, p16(out))
    return out


def checksum(a):
    a = np.ascontiguousarray(a, np.int16)
    return int(lib.orc_checksum(p16(a), a.size))


def lm_head_argmax(table, h):
    table = np.ascontiguousarray(table, np.int16)
    h = np.ascontiguousarray(h, np.int16)
    return int(lib.orc_lm_head_argmax(p16(table), table.shape[0],
                                      table.shape[1], p16(h)))


def shard_words(shape):
    """64-byte words per packed weight shard of a shape."""
    return int(lib.orc_shard_words(ctypes.byref(shape)))


def reference_random_shards(shape, seed, uid=UID_DIVREJ):
    """The reference's 16 packed weight shards for `seed`, each
    [words][32] int16 (initialize_random_model's draw order)."""
    words = shard_words(shape)
    shards = [np.zeros((words, 32), np.int16) for _ in range(16)]
    arr = (_i16p * 16)(*[p16(x) for x in shards])
    rc = lib.orc_reference_random_shards(ctypes.byref(shape), seed, uid,
                                         words, arr)
    assert rc == 0
    return shards


class Model:
    """Row-major fixed-point model held by the oracle."""

    def __init__(self, shape, kept_layers=None, with_embedding=True):
        self.shape = shape
        self.kept = shape.num_layers if kept_layers is None else kept_layers
        self._h = lib.orc_model_create(ctypes.byref(shape), self.kept,
                                       1 if with_embedding else 0)
        self.with_embedding = with_embedding

    def __del__(self):
        h = getattr(self, "_h", None)
        if h:
            lib.orc_model_destroy(h)
            self._h = None

    def _view(self, ptr, count):
        return np.ctypeslib.as_array(ptr, shape=(count,))

    def weight(self, layer, proj):
        s = self.shape
        out_dim = s.intermediate_size if proj in (PROJ_GATE, PROJ_UP) else (
            s.kv_channels if proj in (PROJ_K, PROJ_V) else s.hidden_size)
        in_dim = s.intermediate_size if proj == PROJ_DOWN else s.hidden_size
        ptr = lib.orc_model_weight(self._h, layer, proj)
        return self._view(ptr, out_dim * in_dim).reshape(out_dim, in_dim)

    def norms(self):
        s = self.shape
        return self._view(lib.orc_model_norms(self._h),
                          (2 * s.num_layers + 1) * s.hidden_size).reshape(
                              2 * s.num_layers + 1, s.hidden_size)

    def embedding(self):
        s = self.shape
        assert self.with_embedding
        return self._view(lib.orc_model_embedding(self._h),
                          s.vocab_size * s.hidden_size).reshape(
                              s.vocab_size, s.hidden_size)

    def init_reference_random(self, seed, uid=UID_DIVREJ):
        lib.orc_model_init_reference_random(self._h, seed, uid)

    def load_shards(self, shards):
        """Weights from 16 packed shards, each [words][32] int16."""
        shards = [np.ascontiguousarray(x, np.int16) for x in shards]
        arr = (_i16p * 16)(*[p16(x) for x in shards])
        rc = lib.orc_model_load_shards(self._h, arr, shards[0].size // 32)
        if rc:
            raise ValueError("shards too small for the shape")

    def new_kv(self):
        s = self.shape
        n = s.num_layers * s.num_kv_heads * s.max_seq_len * s.head_dim
        shape = (s.num_layers, s.num_kv_heads, s.max_seq_len, s.head_dim)
        return np.zeros(n, np.int16).reshape(shape), np.zeros(
            n, np.int16).reshape(shape)

    def task(self, kv, op, layer, rows_in, position, token_count=None,
             semantics=SEM_RAW_PAYLOAD):
        kc, vc = kv
        rows_in = np.ascontiguousarray(rows_in, np.int16)
        r = rows_in.shape[0] if token_count is None else token_count
        out = np.zeros((max(r, 1), self.shape.hidden_size), np.int16)
        st = Status()
        code = lib.orc_task(self._h, p16(kc), p16(vc), op, layer, r,
                            position, p16(rows_in), p16(out), semantics,
                            ctypes.byref(st))
        return code, out[:r], st

    def prefill_sequence(self, hidden, layer=0, semantics=SEM_RAW_PAYLOAD):
        hidden = np.ascontiguousarray(hidden, np.int16)
        post = np.zeros_like(hidden)
        out = np.zeros_like(hidden)
        lib.orc_prefill_layer_sequence(self._h, p16(hidden), hidden.shape[0],
                                       layer, semantics, p16(post), p16(out))
        return post, out


def shape(vocab, hidden, inter, layers, heads, kv_heads, max_seq):
    return Shape(vocab, hidden, inter, layers, heads, kv_heads, max_seq)


# Profiles of parse_profile (host:309-343).
PROFILES = {
    "small": (64, 64, 128, 2, 4, 2, 32),
    "medium": (128, 128, 256, 2, 4, 2, 64),
    "qwen-layer": (128, 2048, 11008, 1, 16, 2, 96),
    "qwen-layer-long": (128, 2048, 11008, 1, 16, 2, 2048),
    "qwen2.5-3b": (151936, 2048, 11008, 36, 16, 2, 2048),
}


def profile(name):
    return shape(*PROFILES[name])
