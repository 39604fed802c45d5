"""ctypes binding of libllm_accel.so (the C ABI in include/llm_accel.h).

This is the Python mirror of the reference's accelerator_t boundary
(host/host_qwen_8x64.cpp:1024-2013): a context holding the resident model,
hidden pairs and KV cache, and `task()` = one controller invocation of
Task 16/18/19/20.  Loading fails loudly when the HIP library is missing;
there is no CPU fallback.
"""
import ctypes
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libllm_accel.so")

OP_NOP, OP_DECODER_LAYER = 0, 16
OP_ATTENTION, OP_FFN, OP_FINAL_NORM = 18, 19, 20
# Operator-level ids (include/control_cache_8x64.hpp:253-276), run by op().
(OP_Q_PROJECTION, OP_K_PROJECTION, OP_V_PROJECTION, OP_O_PROJECTION,
 OP_FFN_GATE, OP_FFN_UP, OP_FFN_DOWN, OP_RMSNORM, OP_SILU_MUL,
 OP_RESIDUAL_ADD, OP_ATTN_QK, OP_ATTN_PV, OP_SOFTMAX, OP_ATTN_FLASH,
 OP_DECODE_SMOKE) = range(1, 16)
OP_ATTN_PREFILL_BLOCK = 17
PORT_IN, PORT_AUX, PORT_OUT = 0, 1, 2
ATTENTION_TILE = 64
STATUS_OK, BAD_OPERATOR, BAD_TOKEN_COUNT = 0, 1, 2
BAD_TILE_LENGTH, BAD_POSITION, BAD_LAYER = 3, 4, 5
PROJ_Q, PROJ_K, PROJ_V, PROJ_O, PROJ_GATE, PROJ_UP, PROJ_DOWN = range(7)

_i16p = ctypes.POINTER(ctypes.c_int16)
_u32 = ctypes.c_uint32

# Every symbol include/llm_accel.h declares.
EXPORTS = (
    "llm_ctx_create", "llm_ctx_destroy", "llm_last_error",
    "llm_load_projection", "llm_load_packed_shards", "llm_load_norms",
    "llm_hidden_upload", "llm_hidden_download", "llm_hidden_upload_ports",
    "llm_hidden_download_ports", "llm_task", "llm_kv_read", "llm_kv_write",
    "llm_kv_clear", "llm_pair_device_ptr", "llm_stream", "llm_sync",
    "llm_event_record", "llm_event_elapsed_ms", "llm_exp_tables",
    "llm_kernel_timing", "llm_kernel_stats", "llm_bench_copy",
    "llm_bench_projection", "llm_load_lm_head", "llm_lm_head_argmax",
    "llm_generate", "llm_lm_head_argmax_static", "llm_set_log",
    "llm_load_checkpoint_dir", "llm_op", "llm_port", "llm_port_write",
    "llm_port_read", "llm_weight_bytes",
)
CKPT_TIE_EMBEDDINGS = 1
CKPT_REQUIRE_LM_HEAD = 2
KERNELS = ("rmsnorm", "qkv", "rope", "attention", "oproj", "gateup", "down",
           "attn_sublayer")


class Shape(ctypes.Structure):
    _fields_ = [(n, ctypes.c_uint32) for n in (
        "vocab_size", "hidden_size", "intermediate_size", "num_layers",
        "num_heads", "num_kv_heads", "max_seq_len")] + [
            ("rope_theta", ctypes.c_double)]

    @property
    def head_dim(self):
        return self.hidden_size // self.num_heads

    @property
    def kv_channels(self):
        return self.num_kv_heads * self.head_dim


class Status(ctypes.Structure):
    _fields_ = [(n, ctypes.c_uint32) for n in (
        "op", "code", "token_count", "output_waves", "mm_tasks",
        "vector_tasks", "completed_packets", "last_task")] + [
            ("reserved", ctypes.c_uint32 * 8)]

    def as_tuple(self):
        return (self.op, self.code, self.token_count, self.output_waves,
                self.mm_tasks, self.vector_tasks, self.completed_packets,
                self.last_task)


class GenerateStats(ctypes.Structure):
    _fields_ = [(n, ctypes.c_uint32) for n in (
        "prompt_tokens", "generated_tokens", "prompt_forward_passes",
        "generated_forward_passes", "coarse_task_count",
        "output_materializations", "released_prompt_blocks", "wait_reruns")] + [
            (n, ctypes.c_double) for n in (
                "prompt_forward_ms", "time_to_first_token_ms",
                "generated_forward_ms", "lm_head_ms", "total_ms",
                "generated_wall_ms")] + [
            (n, ctypes.c_uint32) for n in (
                "input_migrations", "output_migrations", "kv_migrations",
                "argmax_readbacks")]

    def as_dict(self):
        return {n: getattr(self, n) for n, _ in self._fields_}


class AccelError(RuntimeError):
    pass


# void (*)(const char* line, void* user)
LOG_FN = ctypes.CFUNCTYPE(None, ctypes.c_char_p, ctypes.c_void_p)


def load_library(path=LIB_PATH):
    if not os.path.exists(path):
        raise AccelError(
            f"{path} is missing: build it with `make -C llm-accel_amd` "
            "(the HIP path has no CPU fallback)")
    lib = ctypes.CDLL(path)
    vp = ctypes.c_void_p
    sig = {
        "llm_ctx_create": (ctypes.c_int, [ctypes.POINTER(Shape), ctypes.c_int,
                                          _u32, ctypes.POINTER(vp)]),
        "llm_ctx_destroy": (None, [vp]),
        "llm_last_error": (ctypes.c_char_p, []),
        "llm_load_projection": (ctypes.c_int, [vp, _u32, _u32, _i16p]),
        "llm_load_packed_shards": (ctypes.c_int, [vp, ctypes.POINTER(_i16p),
                                                  ctypes.c_uint64]),
        "llm_load_norms": (ctypes.c_int, [vp, _i16p]),
        "llm_hidden_upload": (ctypes.c_int, [vp, _u32, _i16p, _u32]),
        "llm_hidden_download": (ctypes.c_int, [vp, _u32, _i16p, _u32]),
        "llm_hidden_upload_ports": (ctypes.c_int, [vp, _u32, _i16p, _i16p,
                                                   _u32, _u32]),
        "llm_hidden_download_ports": (ctypes.c_int, [vp, _u32, _i16p, _i16p,
                                                     _u32, _u32]),
        "llm_task": (ctypes.c_int, [vp, _u32, _u32, _u32, _u32, _u32, _u32,
                                    _u32, ctypes.POINTER(Status)]),
        "llm_kv_read": (ctypes.c_int, [vp, _u32, _u32, _u32, _u32, _i16p,
                                       _i16p]),
        "llm_kv_write": (ctypes.c_int, [vp, _u32, _u32, _u32, _u32, _i16p,
                                        _i16p]),
        "llm_kv_clear": (ctypes.c_int, [vp]),
        "llm_pair_device_ptr": (vp, [vp, _u32]),
        "llm_stream": (vp, [vp]),
        "llm_sync": (ctypes.c_int, [vp]),
        "llm_event_record": (ctypes.c_int, [vp, _u32]),
        "llm_event_elapsed_ms": (ctypes.c_int, [vp, _u32, _u32,
                                                ctypes.POINTER(ctypes.c_float)]),
        "llm_exp_tables": (ctypes.c_int, [_i16p, _i16p]),
        "llm_kernel_timing": (ctypes.c_int, [vp, ctypes.c_int]),
        "llm_kernel_stats": (ctypes.c_int, [vp, _u32,
                                            ctypes.POINTER(ctypes.c_uint64),
                                            ctypes.POINTER(ctypes.c_double)]),
        "llm_bench_copy": (ctypes.c_int, [vp, ctypes.c_uint64, _u32,
                                          ctypes.POINTER(ctypes.c_float)]),
        "llm_bench_projection": (ctypes.c_int, [vp, _u32, _u32, _u32, _u32,
                                                ctypes.POINTER(ctypes.c_float)]),
        "llm_load_lm_head": (ctypes.c_int, [vp, _i16p, _u32]),
        "llm_lm_head_argmax": (ctypes.c_int, [vp, _u32, _u32, _u32,
                                              ctypes.POINTER(ctypes.c_uint32),
                                              ctypes.POINTER(ctypes.c_int64)]),
        "llm_generate": (ctypes.c_int, [vp, _i16p, _u32,
                                        ctypes.POINTER(ctypes.c_uint32), _u32,
                                        _u32, _u32, _u32,
                                        ctypes.POINTER(ctypes.c_uint32),
                                        ctypes.POINTER(GenerateStats)]),
        "llm_lm_head_argmax_static": (ctypes.c_int, [vp, _u32, _u32, vp, _u32,
                                                     _u32, vp, vp, vp]),
        "llm_set_log": (ctypes.c_int, [vp, LOG_FN, vp]),
        "llm_load_checkpoint_dir": (ctypes.c_int, [vp, ctypes.c_char_p, _u32, _i16p]),
        "llm_op": (ctypes.c_int, [vp, _u32, _u32, _u32, _u32, _u32, vp, vp, vp,
                                  ctypes.POINTER(Status)]),
        "llm_port": (ctypes.c_int, [vp, _u32, ctypes.POINTER(vp),
                                    ctypes.POINTER(ctypes.c_size_t)]),
        "llm_port_write": (ctypes.c_int, [vp, _u32, _i16p, ctypes.c_size_t]),
        "llm_port_read": (ctypes.c_int, [vp, _u32, _i16p, ctypes.c_size_t]),
        "llm_weight_bytes": (ctypes.c_int, [vp, ctypes.POINTER(ctypes.c_uint64),
                                            ctypes.POINTER(ctypes.c_uint32)]),
    }
    for name, (res, args) in sig.items():
        f = getattr(lib, name)
        f.restype = res
        f.argtypes = args
    return lib


_lib = None


def lib():
    global _lib
    if _lib is None:
        _lib = load_library()
    return _lib


def _p16(a):
    assert a.dtype == np.int16 and a.flags["C_CONTIGUOUS"]
    return a.ctypes.data_as(_i16p)


def exp_tables():
    a = np.zeros(2049, np.int16)
    b = np.zeros(2049, np.int16)
    lib().llm_exp_tables(_p16(a), _p16(b))
    return a, b


class Accelerator:
    """One device context (mirror of accelerator_t)."""

    def __init__(self, shape, device=0, num_pairs=4):
        self.shape = shape
        self._ctx = ctypes.c_void_p()
        rc = lib().llm_ctx_create(ctypes.byref(shape), device, num_pairs,
                                  ctypes.byref(self._ctx))
        self._check(rc, "llm_ctx_create")

    def close(self):
        if getattr(self, "_ctx", None) and self._ctx.value:
            lib().llm_ctx_destroy(self._ctx)
            self._ctx = ctypes.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    @staticmethod
    def _check(rc, what):
        if rc < 0:
            msg = lib().llm_last_error()
            raise AccelError(f"{what} failed ({rc}): "
                             f"{msg.decode() if msg else ''}")
        return rc

    # --- model ---------------------------------------------------------
    def load_projection(self, layer, proj, w):
        w = np.ascontiguousarray(w, np.int16)
        self._check(lib().llm_load_projection(self._ctx, layer, proj, _p16(w)),
                    "llm_load_projection")

    def load_norms(self, norms):
        norms = np.ascontiguousarray(norms, np.int16)
        self._check(lib().llm_load_norms(self._ctx, _p16(norms)),
                    "llm_load_norms")

    def load_packed_shards(self, shards):
        shards = [np.ascontiguousarray(s, np.int16) for s in shards]
        arr = (_i16p * 16)(*[_p16(s) for s in shards])
        words = shards[0].size // 32
        self._check(lib().llm_load_packed_shards(self._ctx, arr, words),
                    "llm_load_packed_shards")

    def load_model(self, model):
        """model: object with weight(layer, proj) and norms()."""
        for layer in range(self.shape.num_layers):
            for proj in range(7):
                self.load_projection(layer, proj, model.weight(layer, proj))
        self.load_norms(model.norms())

    # --- hidden pairs ---------------------------------------------------
    def upload(self, pair, rows):
        rows = np.ascontiguousarray(rows, np.int16)
        self._check(lib().llm_hidden_upload(self._ctx, pair, _p16(rows),
                                            rows.shape[0]), "upload")

    def download(self, pair, n):
        out = np.zeros((n, self.shape.hidden_size), np.int16)
        self._check(lib().llm_hidden_download(self._ctx, pair, _p16(out), n),
                    "download")
        return out

    def upload_ports(self, pair, port0, port1, rows, stride_words):
        """Rows in the reference's packed feature ports: rows 0-3 in port0,
        rows 4-7 in port1, each row `stride_words` 64-byte words."""
        port0 = np.ascontiguousarray(port0, np.int16)
        port1 = np.ascontiguousarray(port1, np.int16)
        self._check(lib().llm_hidden_upload_ports(
            self._ctx, pair, _p16(port0), _p16(port1), rows, stride_words),
            "upload_ports")

    def download_ports(self, pair, rows, stride_words, port0=None, port1=None):
        n = 4 * stride_words * 32
        port0 = np.zeros(n, np.int16) if port0 is None else port0
        port1 = np.zeros(n, np.int16) if port1 is None else port1
        self._check(lib().llm_hidden_download_ports(
            self._ctx, pair, _p16(port0), _p16(port1), rows, stride_words),
            "download_ports")
        return port0, port1

    # --- LM head and generation ------------------------------------------
    def load_checkpoint_dir(self, path, tie_embeddings=False, require_lm_head=False,
                            want_embedding=True):
        """llm_load_checkpoint_dir; returns the token embedding [vocab][hidden]
        (or None when not wanted)."""
        emb = None
        if want_embedding:
            emb = np.zeros((self.shape.vocab_size, self.shape.hidden_size), np.int16)
        flags = (CKPT_TIE_EMBEDDINGS if tie_embeddings else 0) | \
                (CKPT_REQUIRE_LM_HEAD if require_lm_head else 0)
        self._check(lib().llm_load_checkpoint_dir(
            self._ctx, os.fsencode(path), flags,
            _p16(emb) if emb is not None else None), "llm_load_checkpoint_dir")
        return emb

    def load_lm_head(self, table):
        table = np.ascontiguousarray(table, np.int16)
        self._check(lib().llm_load_lm_head(self._ctx, _p16(table), table.shape[0]),
                    "llm_load_lm_head")

    def lm_head_argmax(self, pair, row0, rows):
        toks = (ctypes.c_uint32 * rows)()
        scores = (ctypes.c_int64 * rows)()
        self._check(lib().llm_lm_head_argmax(self._ctx, pair, row0, rows, toks,
                                             scores), "llm_lm_head_argmax")
        return list(toks), list(scores)

    def generate(self, embedding, prompt, block_size, layer_count, max_new_tokens,
                 log=None):
        """llm_generate; `log`, a list, receives the report lines (the
        forwards are then synchronised one by one)."""
        embedding = np.ascontiguousarray(embedding, np.int16)
        prompt_arr = (ctypes.c_uint32 * len(prompt))(*prompt)
        out = (ctypes.c_uint32 * max(max_new_tokens, 1))()
        st = GenerateStats()
        sink = None
        if log is not None:
            sink = LOG_FN(lambda line, _user: log.append(line.decode()))
            self._check(lib().llm_set_log(self._ctx, sink, None), "llm_set_log")
        try:
            self._check(lib().llm_generate(self._ctx, _p16(embedding), embedding.shape[0],
                                           prompt_arr, len(prompt), block_size,
                                           layer_count, max_new_tokens, out,
                                           ctypes.byref(st)), "llm_generate")
        finally:
            if sink is not None:
                lib().llm_set_log(self._ctx, LOG_FN(), None)
        return list(out)[:max_new_tokens], st.as_dict()

    # --- tasks ------------------------------------------------------------
    def task(self, op, layer, token_count, position, in_pair, out_pair,
             tile_len=0):
        st = Status()
        rc = lib().llm_task(self._ctx, op, layer, token_count, position,
                            tile_len, in_pair, out_pair, ctypes.byref(st))
        self._check(rc, "llm_task")
        return rc, st

    # --- operator-level commands ---------------------------------------
    def port(self, port):
        """(device address, elements) of the context's port buffer."""
        dev = ctypes.c_void_p()
        n = ctypes.c_size_t()
        self._check(lib().llm_port(self._ctx, port, ctypes.byref(dev),
                                   ctypes.byref(n)), "llm_port")
        return dev.value, n.value

    def port_write(self, port, a):
        a = np.ascontiguousarray(a, np.int16).reshape(-1)
        self._check(lib().llm_port_write(self._ctx, port, _p16(a), a.size),
                    "llm_port_write")

    def port_read(self, port, n):
        out = np.zeros(n, np.int16)
        self._check(lib().llm_port_read(self._ctx, port, _p16(out), n),
                    "llm_port_read")
        return out

    def op(self, op, layer=0, token_count=0, position=0, tile_len=0,
           lhs=None, rhs=None, out_elems=0, in_ptr=None, aux_ptr=None,
           out_ptr=None, sync=True):
        """One operator-level command (llm_op).  lhs / rhs go to the
        context's in / aux ports (or device pointers in_ptr / aux_ptr /
        out_ptr are used as given); returns (out_elems values of the out
        port, Status).  A status code != 0 is returned, not raised.  With
        sync=False the work is only enqueued (and nothing is read back)."""
        if lhs is not None:
            self.port_write(PORT_IN, lhs)
        if rhs is not None:
            self.port_write(PORT_AUX, rhs)
        st = Status()
        rc = lib().llm_op(self._ctx, op, layer, token_count, position, tile_len,
                          in_ptr, aux_ptr, out_ptr, ctypes.byref(st))
        self._check(rc, "llm_op")
        if not sync:
            return None, st
        self.sync()
        out = self.port_read(PORT_OUT, out_elems) if out_elems else None
        return out, st

    def _checked(self, op, st):
        if st.code != STATUS_OK:
            raise AccelError(f"controller status failure: op {op} code {st.code}")

    def run_feature(self, op, lhs, rhs=None, layer=0, position=0):
        """run_feature (host/host_qwen_8x64.cpp:1088-1133): projections,
        RMSNorm (rhs = one row of gains), SiLU*up (rhs = up), residual add
        (rhs = the residual rows); lhs [rows][in_dim] -> [rows][out_dim]."""
        sh = self.shape
        h, i, c = sh.hidden_size, sh.intermediate_size, sh.kv_channels
        in_dim = i if op in (OP_FFN_DOWN, OP_SILU_MUL) else h
        out_dim = {OP_K_PROJECTION: c, OP_V_PROJECTION: c, OP_FFN_GATE: i,
                   OP_FFN_UP: i, OP_SILU_MUL: i}.get(op, h)
        lhs = np.ascontiguousarray(lhs, np.int16)
        if lhs.ndim != 2 or not 0 < lhs.shape[0] <= 8 or lhs.shape[1] != in_dim:
            raise AccelError("feature operator input shape mismatch")
        needs_rhs = op in (OP_RMSNORM, OP_SILU_MUL, OP_RESIDUAL_ADD)
        if needs_rhs:
            rows = 1 if op == OP_RMSNORM else lhs.shape[0]
            if rhs is None or np.shape(rhs) != (rows, in_dim):
                raise AccelError("feature operator RHS shape mismatch")
        out, st = self.op(op, layer, lhs.shape[0], position, 0, lhs,
                          rhs if needs_rhs else None, lhs.shape[0] * out_dim)
        self._checked(op, st)
        return out.reshape(lhs.shape[0], out_dim)

    def run_attention(self, op, inputs, aux=None, position=0, tile_len=None,
                      layer=0):
        """run_attention (host/host_qwen_8x64.cpp:1556-1645) over every KV
        head at once: inputs [kv_heads][G][cols] (port k = KV head k).
        aux: K or V panels [kv_heads][tile_len][d] (QK, PV), (k, v) rows
        [kv_heads][d] each (DECODE_SMOKE), None (SOFTMAX, ATTN_FLASH).
        Returns ([kv_heads][G][out_cols], Status)."""
        sh = self.shape
        g, d, hk = sh.num_heads // sh.num_kv_heads, sh.head_dim, sh.num_kv_heads
        src = d if op in (OP_ATTN_QK, OP_ATTN_FLASH, OP_DECODE_SMOKE) else ATTENTION_TILE
        inputs = np.ascontiguousarray(inputs, np.int16)
        if tile_len is None:
            tile_len = 1 if op in (OP_ATTN_FLASH, OP_DECODE_SMOKE) else ATTENTION_TILE
        if inputs.shape != (hk, g, src) or not 0 < tile_len <= ATTENTION_TILE:
            raise AccelError("attention source shape mismatch")
        if op == OP_DECODE_SMOKE:
            k, v = aux
            rhs = np.concatenate([np.asarray(k, np.int16).reshape(-1),
                                  np.asarray(v, np.int16).reshape(-1)])
            if rhs.size != 2 * hk * d:
                raise AccelError("decode smoke KV shape mismatch")
        elif op in (OP_ATTN_QK, OP_ATTN_PV):
            rhs = np.ascontiguousarray(aux, np.int16)
            if rhs.shape != (hk, tile_len, d):
                raise AccelError("attention panel shape mismatch")
        else:
            rhs = None
        cols = {OP_ATTN_QK: ATTENTION_TILE, OP_SOFTMAX: tile_len}.get(op, d)
        out, st = self.op(op, layer, g, position, tile_len, inputs, rhs,
                          hk * g * cols)
        self._checked(op, st)
        return out.reshape(hk, g, cols), st

    def run_prefill_attention_block(self, queries, position, token_count,
                                    layer=0):
        """run_prefill_attention_block (host/host_qwen_8x64.cpp:1647-1675):
        queries [kv_heads][token_count][G][d] -> the same shape."""
        sh = self.shape
        g, d, hk = sh.num_heads // sh.num_kv_heads, sh.head_dim, sh.num_kv_heads
        q = np.ascontiguousarray(queries, np.int16)
        if (not 0 < token_count <= 8 or position + token_count > sh.max_seq_len
                or q.shape != (hk, token_count, g, d)):
            raise AccelError("prefill attention block shape mismatch")
        out, st = self.op(OP_ATTN_PREFILL_BLOCK, layer, token_count, position, 0,
                          q, None, q.size)
        self._checked(OP_ATTN_PREFILL_BLOCK, st)
        return out.reshape(q.shape), st

    # --- KV cache -------------------------------------------------------
    def kv_read(self, layer, kv_head, pos0, n):
        d = self.shape.head_dim
        k = np.zeros((n, d), np.int16)
        v = np.zeros((n, d), np.int16)
        self._check(lib().llm_kv_read(self._ctx, layer, kv_head, pos0, n,
                                      _p16(k), _p16(v)), "kv_read")
        return k, v

    def kv_write(self, layer, kv_head, pos0, k, v):
        k = np.ascontiguousarray(k, np.int16)
        v = np.ascontiguousarray(v, np.int16)
        self._check(lib().llm_kv_write(self._ctx, layer, kv_head, pos0,
                                       k.shape[0], _p16(k), _p16(v)),
                    "kv_write")

    def kv_clear(self):
        self._check(lib().llm_kv_clear(self._ctx), "kv_clear")

    def sync(self):
        self._check(lib().llm_sync(self._ctx), "sync")

    def record(self, slot):
        self._check(lib().llm_event_record(self._ctx, slot), "event_record")

    def kernel_timing(self, enable):
        self._check(lib().llm_kernel_timing(self._ctx, 1 if enable else 0),
                    "kernel_timing")

    def kernel_stats(self):
        """{kernel name: (launches, total_ms)} since timing was enabled."""
        out = {}
        for i, name in enumerate(KERNELS):
            n = ctypes.c_uint64()
            ms = ctypes.c_double()
            self._check(lib().llm_kernel_stats(self._ctx, i, ctypes.byref(n),
                                               ctypes.byref(ms)), "stats")
            out[name] = (n.value, ms.value)
        return out

    def bench_projection(self, kernel, rows, layers, iters):
        us = ctypes.c_float()
        self._check(lib().llm_bench_projection(self._ctx, KERNELS.index(kernel),
                                               rows, layers, iters,
                                               ctypes.byref(us)), "bench_projection")
        return us.value

    def weight_bytes(self):
        """(device bytes of the decoder-layer weight images, matrices held
        in 16 bits)."""
        b = ctypes.c_uint64()
        w = ctypes.c_uint32()
        self._check(lib().llm_weight_bytes(self._ctx, ctypes.byref(b), ctypes.byref(w)),
                    "weight_bytes")
        return b.value, w.value

    def bench_copy(self, nbytes, iters):
        ms = ctypes.c_float()
        self._check(lib().llm_bench_copy(self._ctx, nbytes, iters,
                                         ctypes.byref(ms)), "bench_copy")
        return ms.value

    def elapsed_ms(self, a, b):
        ms = ctypes.c_float()
        self._check(lib().llm_event_elapsed_ms(self._ctx, a, b,
                                               ctypes.byref(ms)), "elapsed")
        return ms.value
