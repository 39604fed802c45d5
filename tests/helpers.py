"""Shared test helpers: build matching oracle / synthetic models."""
import numpy as np

from oracle import orc
import workloads


def oracle_shape(spec, layers=None, max_seq=None):
    return orc.shape(spec.vocab, spec.hidden, spec.inter,
                     spec.layers if layers is None else layers, spec.heads,
                     spec.kv_heads, spec.max_seq if max_seq is None else max_seq)


def accel_shape(spec, layers=None, max_seq=None):
    import llm_accel
    return llm_accel.Shape(spec.vocab, spec.hidden, spec.inter,
                           spec.layers if layers is None else layers,
                           spec.heads, spec.kv_heads,
                           spec.max_seq if max_seq is None else max_seq, 1e6)


def oracle_from_synthetic(synth, shape):
    """Copy a SyntheticModel's arrays into an oracle model."""
    m = orc.Model(shape, shape.num_layers, with_embedding=False)
    for layer in range(shape.num_layers):
        for p in range(7):
            m.weight(layer, p)[:] = synth.weight(layer, p)
    m.norms()[:] = synth.norms()
    return m


def first_mismatch(a, b):
    idx = np.argwhere(a != b)
    if len(idx) == 0:
        return None
    i = tuple(int(v) for v in idx[0])
    return f"{len(idx)} mismatches, first at {i}: got {a[i]} want {b[i]}"
