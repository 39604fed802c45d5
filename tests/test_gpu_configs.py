"""BASELINE configs[2] and configs[4] on the GPU against the CPU oracle.

two Qwen2.5-3B-shaped layers, P16/G8 -- two 8-row prompt
blocks then 7 decode forwards, each sampled token the LM-head argmax of
the last row -- every task's rows and status compared with an oracle
replay, then the whole KV cache of both layers; and llm_generate on the
same request gives the same tokens and task count
(host/host_qwen_8x64.cpp:9016-9136, docs/coarse-task-runtime.md:52-61).

the 36-layer P1024/G128 request runs in full on the GPU; at
the last prompt block and at the last decode forward, layers 0, 17 and 35
are checked against a one-layer oracle step: the layer's input rows and
its K/V cache before the step are taken from the GPU, and the layer's
output rows and the K/V rows it appends must equal the oracle's.  The
oracle has no 36-layer replay here (a full one takes hours at 1 thread).
"""
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


def test_configs2_two_layers_p16_g8_every_task_and_kv():
    import llm_accel
    spec = workloads.CONFIG_B
    layers, P, G, B = 2, 16, 8, 8
    max_seq = 64
    synth = workloads.SyntheticModel(spec, layers=layers)
    head = synth.lm_head()
    emb = synth.embedding()
    prompt = [int(t) for t in synth.tokens(P)]
    om = oracle_from_synthetic(synth, oracle_shape(spec, layers=layers, max_seq=max_seq))
    kv = om.new_kv()
    with llm_accel.Accelerator(accel_shape(spec, layers=layers, max_seq=max_seq)) as acc:
        acc.load_model(synth)
        acc.load_lm_head(head)

        def forward(tokens, pos, final):
            rows = len(tokens)
            cur = emb[tokens].copy()
            acc.upload(1, cur)
            for layer in range(layers):
                for op, pin, pout in ((18, 1, 0), (19, 0, 1)):
                    _say(f"case configs[2] pos={pos} rows={rows} layer={layer} op={op}")
                    code, want, ost = om.task(kv, op, layer, cur, pos)
                    assert code == 0
                    rc, st = acc.task(op, layer, rows, pos, pin, pout)
                    assert rc == 0 and st.as_tuple() == ost.as_tuple()
                    err = first_mismatch(acc.download(pout, rows), want)
                    assert err is None, f"pos {pos} layer {layer} op {op}: {err}"
                    cur = want
            if final:
                code, want, ost = om.task(kv, 20, 0, cur, pos)
                rc, st = acc.task(20, 0, rows, pos, 1, 0)
                assert rc == 0 and st.as_tuple() == ost.as_tuple()
                err = first_mismatch(acc.download(0, rows), want)
                assert err is None, f"pos {pos} final norm: {err}"
                cur = want
            return cur

        forward(prompt[0:8], 0, False)
        fin = forward(prompt[8:16], 8, True)
        tokens = []
        for step in range(G):
            want_tok = orc.lm_head_argmax(head, fin[-1])
            got_tok, _ = acc.lm_head_argmax(0, fin.shape[0] - 1, 1)
            assert got_tok[0] == want_tok, f"step {step}"
            tokens.append(want_tok)
            if step + 1 < G:
                fin = forward([want_tok], P + step, True)
        n = P + G - 1
        for layer in range(layers):
            for h in range(spec.kv_heads):
                gk, gv = acc.kv_read(layer, h, 0, n)
                assert np.array_equal(gk, kv[0][layer, h, :n]), (layer, h)
                assert np.array_equal(gv, kv[1][layer, h, :n]), (layer, h)

        # the same request through the library's own generate loop
        acc.kv_clear()
        _say("case configs[2] llm_generate")
        toks, st = acc.generate(emb, prompt, B, layers, G)
        assert toks == tokens
        assert st["coarse_task_count"] == 2 * 2 * layers + 1 + (G - 1) * (2 * layers + 1)
        for layer in range(layers):
            for h in range(spec.kv_heads):
                gk, gv = acc.kv_read(layer, h, 0, n)
                assert np.array_equal(gk, kv[0][layer, h, :n])
                assert np.array_equal(gv, kv[1][layer, h, :n])


def _one_layer_oracle(synth, spec, layer, layers, max_seq):
    """Oracle model of layer `layer` alone: its weights, its two norm rows
    and the final norm row."""
    shape = oracle_shape(spec, layers=1, max_seq=max_seq)
    m = orc.Model(shape, 1, with_embedding=False)
    for p in range(7):
        m.weight(0, p)[:] = synth.weight(layer, p)
    norms = synth.norms()
    m.norms()[0] = norms[2 * layer]
    m.norms()[1] = norms[2 * layer + 1]
    m.norms()[2] = norms[2 * layers]
    return m


def test_configs4_36_layers_p1024_g128_checked_layers():
    import llm_accel
    spec = workloads.CONFIG_B
    layers, P, G, B = 36, 1024, 128, 8
    max_seq = P + G
    checked = (0, 17, 35)
    _say("building 36 synthetic layers")
    synth = workloads.SyntheticModel(spec, layers=layers)
    head = synth.lm_head()
    emb = synth.embedding()
    prompt = [int(t) for t in synth.tokens(P)]
    oracles = {l: _one_layer_oracle(synth, spec, l, layers, max_seq) for l in checked}
    with llm_accel.Accelerator(accel_shape(spec, layers=layers, max_seq=max_seq)) as acc:
        acc.load_model(synth)
        acc.load_lm_head(head)

        def check_layer(layer, rows, pos):
            """Before T18 of `layer`: its input rows are in pair 1."""
            x = acc.download(1, rows)
            m = oracles[layer]
            okv = m.new_kv()
            for h in range(spec.kv_heads):
                if pos:
                    k, v = acc.kv_read(layer, h, 0, pos)
                    okv[0][0, h, :pos] = k
                    okv[1][0, h, :pos] = v
            _, mid, _ = m.task(okv, 18, 0, x, pos)
            _, out, _ = m.task(okv, 19, 0, mid, pos)
            return out, okv

        def forward(tokens, pos, final, check):
            rows = len(tokens)
            acc.upload(1, emb[tokens])
            for layer in range(layers):
                want = None
                if check and layer in checked:
                    _say(f"case configs[4] pos={pos} rows={rows} layer={layer}")
                    want, okv = check_layer(layer, rows, pos)
                rc, _ = acc.task(18, layer, rows, pos, 1, 0)
                assert rc == 0
                rc, _ = acc.task(19, layer, rows, pos, 0, 1)
                assert rc == 0
                if want is not None:
                    err = first_mismatch(acc.download(1, rows), want)
                    assert err is None, f"pos {pos} layer {layer}: {err}"
                    for h in range(spec.kv_heads):
                        k, v = acc.kv_read(layer, h, pos, rows)
                        assert np.array_equal(k, okv[0][0, h, pos:pos + rows]), (layer, h)
                        assert np.array_equal(v, okv[1][0, h, pos:pos + rows]), (layer, h)
            if final:
                rc, _ = acc.task(20, 0, rows, pos, 1, 0)
                assert rc == 0

        for b0 in range(0, P, B):
            forward(prompt[b0:b0 + B], b0, b0 + B == P, b0 + B == P)
        last = B - 1
        for step in range(G):
            tok, _ = acc.lm_head_argmax(0, last, 1)
            last = 0
            if step + 1 < G:
                forward([tok[0]], P + step, True, step + 2 == G)
        # the last sampled token against the oracle argmax of the final row
        fin = acc.download(0, 1)
        assert tok[0] == orc.lm_head_argmax(head, fin[0])
