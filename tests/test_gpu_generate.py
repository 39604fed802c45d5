"""Device LM-head argmax and the generate driver on the GPU.

The argmax restates model_data_t::lm_head_argmax (host/host_qwen_8x64.cpp
:937-969): exact int64 scores, strict > scan, first index on ties.  The
generate driver restates the reference's coarse-task generate loop
(host/host_qwen_8x64.cpp:9016-9136): prompt blocks, Task 20 only after the
final block, one forward per sampled token but the last; its task count is
ceil(P/B)*2L + 1 + (G-1)*(2L+1) (docs/coarse-task-runtime.md:52-61).  The
Qwen2.5-3B one- and two-layer generations reproduce the reference's
published sampled tokens (KAT-2/3)."""
import json
import os
import sys

import numpy as np
import pytest

from oracle import orc
import workloads
from helpers import accel_shape, oracle_from_synthetic, oracle_shape

pytestmark = pytest.mark.gpu

HERE = os.path.dirname(os.path.abspath(__file__))
KAT = json.load(open(os.path.join(HERE, "golden", "kat.json")))


def _say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def test_lm_head_argmax_matches_oracle_and_ties():
    import llm_accel
    spec = workloads.CONFIG_A
    synth = workloads.SyntheticModel(spec, layers=1)
    table = synth.embedding().copy()
    rng = np.random.default_rng(7)
    rows = rng.integers(-32768, 32768, (8, spec.hidden), dtype=np.int16)
    # a duplicated best row: the first copy must win
    table[900] = table[17] = rng.integers(100, 128, spec.hidden, dtype=np.int16)
    rows[5] = 120
    with llm_accel.Accelerator(accel_shape(spec, layers=1, max_seq=64)) as a:
        a.load_model(synth)
        a.load_lm_head(table)
        a.upload(2, rows)
        _say("case lm-head argmax config A")
        toks, scores = a.lm_head_argmax(2, 0, 8)
        toks3, _ = a.lm_head_argmax(2, 5, 3)
    want = [orc.lm_head_argmax(table, rows[r]) for r in range(8)]
    assert toks == want
    assert toks[5] == 17
    assert toks3 == want[5:8]
    direct = rows.astype(np.int64) @ table.astype(np.int64).T
    assert scores == [int(direct[r, toks[r]]) for r in range(8)]


def test_lm_head_argmax_full_vocabulary():
    import llm_accel
    spec = workloads.CONFIG_B
    synth = workloads.SyntheticModel(spec, layers=1)
    table = synth.embedding()
    h = synth.hidden_rows(2)
    with llm_accel.Accelerator(accel_shape(spec, layers=1, max_seq=64)) as a:
        a.load_lm_head(table)
        a.upload(0, h)
        _say("case lm-head argmax vocab 151936")
        toks, _ = a.lm_head_argmax(0, 0, 2)
    assert toks == [orc.lm_head_argmax(table, h[r]) for r in range(2)]


def test_generate_matches_oracle_replay():
    import llm_accel
    spec = workloads.CONFIG_A
    layers = 2
    synth = workloads.SyntheticModel(spec, layers=layers)
    emb = synth.embedding()
    prompt = [int(t) for t in synth.tokens(13)]
    G, B = 4, 8
    with llm_accel.Accelerator(accel_shape(spec, layers=layers, max_seq=64)) as a:
        a.load_model(synth)
        a.load_lm_head(emb)
        _say("case generate config A P13/G4 B8")
        toks, st = a.generate(emb, prompt, B, layers, G)
    om = oracle_from_synthetic(synth, oracle_shape(spec, layers=layers, max_seq=64))
    kv = om.new_kv()

    def forward(rows, pos, final):
        h = emb[rows].copy()
        for layer in range(layers):
            _, h, _ = om.task(kv, 18, layer, h, pos)
            _, h, _ = om.task(kv, 19, layer, h, pos)
        if final:
            _, h, _ = om.task(kv, 20, 0, h, pos)
        return h

    h = forward(prompt[0:8], 0, False)
    h = forward(prompt[8:13], 8, True)
    want = []
    for step in range(G):
        t = orc.lm_head_argmax(emb, h[-1])
        want.append(t)
        if step + 1 < G:
            h = forward([t], 13 + step, True)
    assert toks == want
    assert st["coarse_task_count"] == 2 * 2 * layers + 1 + (G - 1) * (2 * layers + 1)
    assert st["prompt_forward_passes"] == 2 and st["released_prompt_blocks"] == 1
    assert st["generated_forward_passes"] == G - 1
    assert st["output_materializations"] == G


@pytest.fixture(scope="module")
def qwen3b_reference_model():
    # initialize_random_model(20260718) on the qwen2.5-3b profile, layers 0-1
    _say("building the reference random Qwen2.5-3B model (layers 0-1)")
    m = orc.Model(orc.profile("qwen2.5-3b"), 2, True)
    m.init_reference_random(20260718, orc.UID_DIVREJ)
    return m


@pytest.mark.parametrize("layers,kat", [(1, "kat2_qwen3b_l1"), (2, "kat3_qwen3b_l2")])
def test_kat2_kat3_generated_tokens(qwen3b_reference_model, layers, kat):
    """Prompt tokens 0..7 as one block of 8, two sampled tokens, tied LM
    head: the reference's published generations
    (results/qwen3b-e2e-20260820, results/qwen3b-e2e-l2-20260821)."""
    import llm_accel
    m = qwen3b_reference_model
    s = orc.profile("qwen2.5-3b")
    shape = llm_accel.Shape(s.vocab_size, s.hidden_size, s.intermediate_size,
                            s.num_layers, s.num_heads, s.num_kv_heads, 64, 1e6)
    k = KAT[kat]
    with llm_accel.Accelerator(shape) as a:
        for layer in range(layers):
            for p in range(7):
                a.load_projection(layer, p, m.weight(layer, p))
        a.load_norms(m.norms())
        a.load_lm_head(m.embedding())
        _say(f"case {kat} generate")
        toks, st = a.generate(m.embedding(), k["prompt"], 8, layers, 2)
    assert toks == k["generated"]
    assert st["coarse_task_count"] == 2 * layers + 1 + (2 * layers + 1)
