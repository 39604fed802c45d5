"""The C-ABI library: loads, exports every function include/llm_accel.h
declares, and fails loudly (no CPU fallback) when no GPU is present."""
import ctypes
import os
import re

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "llm_accel.h")


def _declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(llm_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_the_boundary():
    names = _declared_functions()
    for required in ("llm_ctx_create", "llm_task", "llm_hidden_upload",
                     "llm_hidden_download", "llm_kv_read", "llm_kv_write",
                     "llm_load_packed_shards"):
        assert required in names


def test_library_exports_every_declared_symbol():
    import llm_accel
    lib = ctypes.CDLL(llm_accel.LIB_PATH)
    missing = [n for n in _declared_functions() if not hasattr(lib, n)]
    assert not missing
    assert sorted(llm_accel.EXPORTS) == _declared_functions()


def test_context_creation_fails_loudly_without_gpu():
    import llm_accel
    shape = llm_accel.Shape(64, 256, 688, 1, 4, 2, 64, 1e6)
    try:
        acc = llm_accel.Accelerator(shape)
    except llm_accel.AccelError as e:
        assert "device" in str(e).lower() or "hip" in str(e).lower()
        return
    acc.close()
    pytest.skip("a GPU is present; this checks the no-GPU path")


def test_bad_shapes_are_rejected_before_device_use():
    import llm_accel
    lib = llm_accel.lib()
    ctx = ctypes.c_void_p()
    for args in ((64, 250, 688, 1, 4, 2, 64), (64, 256, 688, 1, 3, 2, 64),
                 (64, 4096, 688, 1, 8, 2, 64), (64, 256, 688, 0, 4, 2, 64)):
        shape = llm_accel.Shape(*args, 1e6)
        rc = lib.llm_ctx_create(ctypes.byref(shape), 0, 2, ctypes.byref(ctx))
        assert rc == -1, args
        assert lib.llm_last_error()


def test_workloads_are_deterministic():
    import workloads
    a = workloads.SyntheticModel(workloads.CONFIG_A, layers=1)
    b = workloads.SyntheticModel(workloads.CONFIG_A, layers=1)
    for p in range(7):
        assert np.array_equal(a.weight(0, p), b.weight(0, p))
    w = a.weight(0, 0)
    assert w.dtype == np.int16 and w.min() >= -1024 and w.max() <= 1024
    g = a.norms()
    assert g.min() >= 128 and g.max() <= 384
    assert a.weight(0, 6).shape == (256, 688)
