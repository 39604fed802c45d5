"""On-disk packed Fix16 checkpoints (model_data_t::load,
host/host_qwen_8x64.cpp:736-840): the reference random model written in
the reference's file layout (16 packed weight shards, norm table,
embedding, optional LM head) loads through llm_load_checkpoint_dir and
then matches the oracle's model task for task; every file must have
exactly its expected size, and the reference's error text names it."""
import os
import sys

import numpy as np
import pytest

from oracle import orc

pytestmark = pytest.mark.gpu

SEED = 20260718


def _say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def _write(d, model, shards, lm_head=None):
    model.embedding().tofile(os.path.join(d, "token_embedding.fix16.bin"))
    model.norms().tofile(os.path.join(d, "norm_weights.fix16.bin"))
    for i, sh in enumerate(shards):
        sh.tofile(os.path.join(d, f"layer_weights_shard{i:02d}.fix16.bin"))
    if lm_head is not None:
        lm_head.tofile(os.path.join(d, "lm_head.fix16.bin"))


def _shape(llm_accel, s):
    return llm_accel.Shape(s.vocab_size, s.hidden_size, s.intermediate_size,
                           s.num_layers, s.num_heads, s.num_kv_heads, s.max_seq_len, 1e6)


@pytest.fixture(scope="module")
def reference_model():
    s = orc.profile("medium")
    m = orc.Model(s)
    m.init_reference_random(SEED)
    shards = orc.reference_random_shards(s, SEED)
    lm_head = np.random.default_rng(5).integers(-128, 129, (s.vocab_size, s.hidden_size),
                                                dtype=np.int16)
    return s, m, shards, lm_head


def _forward_matches(acc, s, m, table):
    """P8 through every layer, Task 20, LM-head argmax of every row, then a
    decode row: against the oracle model."""
    kv = m.new_kv()
    h = m.embedding()[0:8].copy()
    acc.upload(1, h)
    cur = h
    for layer in range(s.num_layers):
        for op, pin, pout in ((18, 1, 0), (19, 0, 1)):
            rc, _ = acc.task(op, layer, 8, 0, pin, pout)
            assert rc == 0
            _, cur, _ = m.task(kv, op, layer, cur, 0)
            assert np.array_equal(acc.download(pout, 8), cur), (op, layer)
    acc.task(20, 0, 8, 0, 1, 0)
    _, fin, _ = m.task(kv, 20, 0, cur, 0)
    assert np.array_equal(acc.download(0, 8), fin)
    toks, _ = acc.lm_head_argmax(0, 0, 8)
    assert toks == [orc.lm_head_argmax(table, fin[r]) for r in range(8)]


def test_checkpoint_dir_round_trip(tmp_path, reference_model):
    import llm_accel
    s, m, shards, lm_head = reference_model
    _write(str(tmp_path), m, shards, lm_head)
    with llm_accel.Accelerator(_shape(llm_accel, s)) as acc:
        _say("case checkpoint dir: untied LM head")
        emb = acc.load_checkpoint_dir(str(tmp_path), require_lm_head=True)
        assert np.array_equal(emb, m.embedding())
        _forward_matches(acc, s, m, lm_head)
    os.remove(os.path.join(tmp_path, "lm_head.fix16.bin"))
    with llm_accel.Accelerator(_shape(llm_accel, s)) as acc:
        _say("case checkpoint dir: tied embeddings")
        assert acc.load_checkpoint_dir(str(tmp_path), tie_embeddings=True,
                                       want_embedding=False) is None
        _forward_matches(acc, s, m, m.embedding())


def test_checkpoint_dir_exact_sizes(tmp_path, reference_model):
    import llm_accel
    s, m, shards, lm_head = reference_model
    _write(str(tmp_path), m, shards, lm_head)
    words = orc.shard_words(s)
    with llm_accel.Accelerator(_shape(llm_accel, s)) as acc:
        _say("case checkpoint dir: size checks")
        # one shard 64 bytes short
        p5 = os.path.join(tmp_path, "layer_weights_shard05.fix16.bin")
        shards[5][:-1].tofile(p5)
        with pytest.raises(llm_accel.AccelError) as e:
            acc.load_checkpoint_dir(str(tmp_path))
        msg = str(e.value)
        assert "weight shard size mismatch: " in msg and p5 in msg
        assert f"expected={words * 64}" in msg and f"actual={(words - 1) * 64}" in msg
        shards[5].tofile(p5)
        # embedding one value too long
        pe = os.path.join(tmp_path, "token_embedding.fix16.bin")
        np.concatenate([m.embedding().ravel(), [0]]).astype(np.int16).tofile(pe)
        with pytest.raises(llm_accel.AccelError) as e:
            acc.load_checkpoint_dir(str(tmp_path))
        assert "embedding size mismatch: " in str(e.value)
        m.embedding().tofile(pe)
        # a missing norm table reads as size 0
        pn = os.path.join(tmp_path, "norm_weights.fix16.bin")
        os.remove(pn)
        with pytest.raises(llm_accel.AccelError) as e:
            acc.load_checkpoint_dir(str(tmp_path))
        assert "norm weights size mismatch: " in str(e.value) and "actual=0" in str(e.value)
        m.norms().tofile(pn)
        # no LM head file, not tied, required
        os.remove(os.path.join(tmp_path, "lm_head.fix16.bin"))
        with pytest.raises(llm_accel.AccelError) as e:
            acc.load_checkpoint_dir(str(tmp_path), require_lm_head=True)
        assert "lm_head.fix16.bin" in str(e.value)
        # a wrong-size LM head is rejected too
        lm_head[:-1].tofile(os.path.join(tmp_path, "lm_head.fix16.bin"))
        with pytest.raises(llm_accel.AccelError) as e:
            acc.load_checkpoint_dir(str(tmp_path))
        assert "LM head size mismatch: " in str(e.value)
        # and after the failures a good directory still loads
        lm_head.tofile(os.path.join(tmp_path, "lm_head.fix16.bin"))
        acc.load_checkpoint_dir(str(tmp_path), require_lm_head=True)
        _forward_matches(acc, s, m, lm_head)
