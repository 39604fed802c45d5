"""Benchmark of the resident decoder-layer path on one MI355X.

Workload: one Qwen2.5-3B-shaped decoder layer
(hidden 2048, 16 query / 2 KV heads of 128, SwiGLU 11008), P8/G2: one
8-row prefill block (Task 18 -> 19 -> 20 at position 0) then one
single-row decode forward (Task 18 -> 19 -> 20 at position 8).  The LM-head
argmax stays on the host and outside the timed region, as in the
reference's decode_token_s (host/host_qwen_8x64.cpp:9265-9273).

A step is one such P8/G2 pass over one layer.  The context holds
`--copies` distinct weight copies of the layer and step s uses copy
s % copies, so the streamed working set (8 x 154 MB by default) exceeds
the 256 MB Infinity Cache and the measured bandwidth is HBM bandwidth.
The timed region runs the K prefill blocks, then the K decode forwards.
Inputs (prompt rows, decode row) are resident in HBM before timing.

Prints one JSON line.  `value` = decode forwards per second of the layer.
"""
import argparse
import json
import os
import platform
import subprocess
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)
sys.path.insert(0, os.path.join(ROOT, "llm-accel_amd"))

import numpy as np  # noqa: E402

METRIC = ("decode tok/s + P8 prefill block µs, Qwen2.5-3B shape; "
          "% of HBM roofline")
HBM_PEAK_GBS = 8000.0  # MI355X published HBM3E bandwidth


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--copies", type=int, default=8)
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--sweep", action=argparse.BooleanOptionalAction, default=True,
                    help="configs[3] decode context sweep (extra field)")
    ap.add_argument("--full", action=argparse.BooleanOptionalAction, default=True,
                    help="configs[2] and configs[4] request loops (extra fields)")
    return ap.parse_args()


def layer_bytes(spec):
    return spec.weight_bytes_per_layer()


def gateup_bytes(spec, rows):
    """Algorithmic HBM bytes of one gate|up + SiLU*up launch: both weight
    matrices once, the normalised input rows, the product rows written."""
    h, i = spec.hidden, spec.inter
    return 2 * (2 * i * h) + 2 * rows * h + 2 * rows * i


def cpu_model_name():
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or "unknown"


def load_traffic():
    """HBM bytes per decode gate|up launch measured with rocprofv3 PMC
    counters (profiles/gateup_decode_traffic.md), or None."""
    path = os.path.join(ROOT, "profiles", "gateup_decode_traffic.md")
    try:
        for line in open(path):
            if line.startswith("traffic_bytes_per_launch:"):
                return float(line.split(":", 1)[1])
    except OSError:
        pass
    return None


def cpu_baseline(spec, synth, seconds):
    """The oracle (single thread) on a bounded sample of the same workload:
    P8 blocks and decode forwards of layer copy 0, for about `seconds`."""
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    from oracle import orc
    from helpers import oracle_from_synthetic, oracle_shape
    orc.lib.orc_set_threads(1)
    om = oracle_from_synthetic(synth, oracle_shape(spec, layers=1, max_seq=64))
    kv = om.new_kv()
    prompt = synth.hidden_rows(8)
    row = synth.hidden_rows(9)[8:9]
    p8_times, dec_times = [], []
    t_end = time.perf_counter() + seconds
    while True:
        t0 = time.perf_counter()
        _, x, _ = om.task(kv, 18, 0, prompt, 0)
        _, x, _ = om.task(kv, 19, 0, x, 0)
        om.task(kv, 20, 0, x, 0)
        t1 = time.perf_counter()
        _, x, _ = om.task(kv, 18, 0, row, 8)
        _, x, _ = om.task(kv, 19, 0, x, 8)
        om.task(kv, 20, 0, x, 8)
        t2 = time.perf_counter()
        p8_times.append(t1 - t0)
        dec_times.append(t2 - t1)
        if t2 > t_end:
            break
    dec = float(np.mean(dec_times))
    return {
        "value": 1.0 / dec,
        "unit": "decode tok/s (1 Qwen2.5-3B-shaped layer)",
        "cores": 1,
        "kind": "port",
        "sample": (f"{len(dec_times)} x (P8 block + decode forward) of "
                   f"configs[1] layer copy 0, oracle C restatement, 1 thread "
                   f"on {cpu_model_name()} ({os.cpu_count()} host threads)"),
        "p8_block_us": float(np.mean(p8_times)) * 1e6,
        "decode_forward_us": dec * 1e6,
    }


def load_copies(acc, synth, copies):
    """`copies` distinct copies of synth's layer 0 as layers 0..copies-1:
    copy c permutes the columns of every matrix by c (same bytes per
    matrix, different addresses and values)."""
    for c in range(copies):
        for p in range(7):
            w = synth.weight(0, p)
            acc.load_projection(c, p, w if c == 0 else np.roll(w, c, axis=1))
    acc.load_norms(np.concatenate([np.tile(synth.norms()[:2], (copies, 1)),
                                   synth.norms()[2:3]]))


def context_sweep(llm_accel, workloads, spec, synth, copies=4):
    """one layer, K/V preloaded with seeded Q8.8
    N(0, 0.3) to n positions, one decode forward (T18/T19/T20) at position
    n.  The context holds `copies` copies of the layer, each with its own
    K/V cache, and the forwards rotate over them, so that every forward
    finds its weights and K/V evicted by the others (4 x (154 MB + K/V) >
    the 256 MB Infinity Cache) without a flush kernel's dirty lines being
    written back during it; median of 8 forwards after 4 warm-up ones."""
    nmax = 16384
    shape = llm_accel.Shape(spec.vocab, spec.hidden, spec.inter, copies, spec.heads,
                            spec.kv_heads, nmax + 64, 1e6)
    out = {}
    with llm_accel.Accelerator(shape, num_pairs=4) as a:
        load_copies(a, synth, copies)
        for h in range(spec.kv_heads):
            k, v = synth.kv_rows(nmax, seed_offset=20 + h)
            for c in range(copies):
                a.kv_write(c, h, 0, k, v)
        a.upload(3, synth.hidden_rows(1))
        for n in (128, 1024, 4096, 16384):
            times = []
            for rep in range(12):
                layer = rep % copies
                a.record(0)
                a.task(18, layer, 1, n, 3, 0)
                a.task(19, layer, 1, n, 0, 1)
                a.task(20, 0, 1, n, 1, 0)
                a.record(1)
                a.sync()
                if rep >= 4:
                    times.append(a.elapsed_ms(0, 1) * 1e3)
            out[str(n)] = round(float(np.median(times)), 2)
    return out


def request_loop(llm_accel, workloads, spec, layers, prompt_len, gen, emb, lm_head):
    """`layers` Qwen2.5-3B-shaped layers
    (seeded synthetic weights, embedding and LM head), the reference's
    generate loop through llm_generate: the prompt in 8-row blocks through
    every layer (Task 18 / 19 per layer, Task 20 after the last block), then
    `gen` sampled tokens, each the device LM-head argmax of the last row
    with a one-row forward for every token but the last; hidden state and
    KV cache stay in HBM throughout.  decode tok/s = generated forwards /
    their time, LM head excluded (decode_token_s, host/host_qwen_8x64.cpp
    :9265-9273); times are host clocks around each forward, as the
    reference reports them.  The request runs 3 times after a short
    warm-up one; the figures are those of the run with the median total
    time (a request occasionally meets a host-side stall of a few ms,
    which would dominate the 2-layer configs[2])."""
    runs = 3
    t0 = time.perf_counter()
    s = workloads.with_layers(spec, layers, max_seq=prompt_len + gen)
    synth = workloads.SyntheticModel(s)
    shape = llm_accel.Shape(spec.vocab, spec.hidden, spec.inter, layers,
                            spec.heads, spec.kv_heads, prompt_len + gen, 1e6)
    with llm_accel.Accelerator(shape, num_pairs=4) as a:
        a.load_model(synth)
        prompt = [int(t) for t in synth.tokens(prompt_len)]
        del synth
        a.load_lm_head(lm_head)
        setup_s = time.perf_counter() - t0
        # one short warm-up request (kernels, page tables), then the runs
        a.generate(emb, prompt[:8], 8, layers, 2)
        results = sorted((a.generate(emb, prompt, 8, layers, gen) for _ in range(runs)),
                         key=lambda r: r[1]["total_ms"])
        toks, st = results[runs // 2]
        assert all(r[0] == toks for r in results), "runs generated different tokens"
    dec_ms = st["generated_forward_ms"] / max(st["generated_forward_passes"], 1)
    blocks = st["prompt_forward_passes"]
    kv_bytes = 4 * spec.kv_heads * spec.head_dim * (prompt_len + gen / 2)
    return {
        "workload": f"{layers} layers, P{prompt_len}/G{gen}, 8-row prompt blocks, "
                    "device LM-head argmax",
        "decode_tok_s": 1e3 / dec_ms,
        "decode_forward_ms": dec_ms,
        "decode_hbm_frac": layers * (layer_bytes(spec) + kv_bytes) / (dec_ms * 1e-3)
                           / 1e9 / HBM_PEAK_GBS,
        "prompt_ms": st["prompt_forward_ms"],
        "p8_block_us_per_layer": st["prompt_forward_ms"] * 1e3 / (blocks * layers),
        "time_to_first_token_ms": st["time_to_first_token_ms"],
        "lm_head_ms_per_token": st["lm_head_ms"] / max(st["generated_tokens"], 1),
        "total_ms": st["total_ms"],
        "coarse_tasks": st["coarse_task_count"],
        "first_tokens": toks[:4],
        "setup_s": round(setup_s, 1),
    }


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py: this build targets one GPU; --gpus {args.gpus} is "
              "not supported (the sharded design is described in DESIGN.md)",
              file=sys.stderr)
        sys.exit(2)
    import llm_accel
    import workloads
    spec = workloads.CONFIG_B
    C = args.copies
    synth = workloads.SyntheticModel(spec, layers=1)
    shape = llm_accel.Shape(spec.vocab, spec.hidden, spec.inter, C, spec.heads,
                            spec.kv_heads, 64, 1e6)
    acc = llm_accel.Accelerator(shape, num_pairs=4)
    load_copies(acc, synth, C)
    prompt = synth.hidden_rows(8)
    row = synth.hidden_rows(9)[8:9]
    acc.upload(2, prompt)
    acc.upload(3, row)

    def step(layer):
        acc.task(18, layer, 8, 0, 2, 0)
        acc.task(19, layer, 8, 0, 0, 1)
        acc.task(20, 0, 8, 0, 1, 0)

    def decode(layer):
        acc.task(18, layer, 1, 8, 3, 0)
        acc.task(19, layer, 1, 8, 0, 1)
        acc.task(20, 0, 1, 8, 1, 0)

    for s in range(args.warmup):
        step(s % C)
        decode(s % C)
    acc.sync()

    # K steps = K prefill blocks then K decode forwards, each rotating over
    # the copies, so no block or forward finds its weights cached by the
    # one before it (P8 and decode read different layouts of a copy).
    K = args.steps
    assert 2 * K + 2 <= 1024
    acc.sync()
    t_host0 = time.perf_counter()
    for s in range(K):
        acc.record(s)
        step(s % C)
    acc.record(K)
    for s in range(K):
        acc.record(K + 1 + s)
        decode(s % C)
    acc.record(2 * K + 1)
    acc.sync()
    t_host1 = time.perf_counter()
    total_ms = acc.elapsed_ms(0, 2 * K + 1) - acc.elapsed_ms(K, K + 1)
    p8 = [acc.elapsed_ms(s, s + 1) for s in range(K)]
    dec = [acc.elapsed_ms(K + 1 + s, K + 2 + s) for s in range(K)]
    p8_us = float(np.median(p8)) * 1e3
    dec_us = float(np.median(dec)) * 1e3

    # Per-kernel pass: decode forwards, then P8 blocks, kernel events on.
    def kernel_pass(fn):
        acc.kernel_timing(True)
        for s in range(K):
            fn(s % C)
        stats = acc.kernel_stats()
        acc.kernel_timing(False)
        return {k: (n, ms / n * 1e3 if n else 0.0) for k, (n, ms) in stats.items()}

    kdec = kernel_pass(decode)
    kp8 = kernel_pass(step)
    # Host-inclusive decode forward: row upload, T18/T19/T20, row download
    # (the reference's decode path moves one row each way over PCIe).
    io = []
    for s in range(K):
        t0 = time.perf_counter()
        acc.upload(3, row)
        decode(s % C)
        acc.download(0, 1)
        io.append(time.perf_counter() - t0)
    dec_io_us = float(np.median(io)) * 1e6
    # The dominant kernel back to back (same launches as in a decode
    # forward, rotating the layer copies): its mean launch duration.
    gu_us = acc.bench_projection("gateup", 1, C, 4 * K)

    copy_bytes = 512 << 20
    copy_ms = acc.bench_copy(copy_bytes, 20)
    copy_gbs = 2 * copy_bytes / copy_ms / 1e6
    acc.close()
    sweep = context_sweep(llm_accel, workloads, spec, synth) if args.sweep else None
    full = None
    if args.full:
        # seeded embedding table and LM head [151936][2048], shared by both
        tables = workloads.SyntheticModel(workloads.with_layers(spec, 0))
        emb, lm_head = tables.embedding(), tables.lm_head()
        full = {
            "configs[2]": request_loop(llm_accel, workloads, spec, 2, 16, 8, emb, lm_head),
            "configs[4]": request_loop(llm_accel, workloads, spec, 36, 1024, 128,
                                       emb, lm_head),
        }
        del emb, lm_head

    lb = layer_bytes(spec)
    gu_bytes = gateup_bytes(spec, 1)
    achieved = gu_bytes / (gu_us * 1e-6) / 1e9
    traffic = load_traffic()
    out = {
        "metric": METRIC,
        "value": 1e6 / dec_us,
        "unit": "decode tok/s (1 Qwen2.5-3B-shaped layer)",
        "n_gpus": 1,
        "steps": K,
        "warmup": args.warmup,
        "ms_per_step": total_ms / K,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int16",
        "data": "synthetic",
        "config": {
            "workload": ("configs[1]: one Qwen2.5-3B-shaped decoder layer "
                         "(H 2048, 16/2 heads x 128, I 11008), P8/G2 = one "
                         "8-row prefill block + one decode forward, Task "
                         "18/19/20, host LM head excluded"),
            "layer_copies": C,
            "weight_bytes_per_layer": lb,
            "seed": workloads.SEED,
        },
        "p8_block_us": p8_us,
        "decode_forward_us": dec_us,
        "decode_hbm_frac": lb / (dec_us * 1e-6) / 1e9 / HBM_PEAK_GBS,
        "p8_hbm_frac": lb / (p8_us * 1e-6) / 1e9 / HBM_PEAK_GBS,
        "host_wall_ms_per_step": (t_host1 - t_host0) * 1e3 / K,
        "decode_forward_with_host_io_us": dec_io_us,
        "kernel_us_decode": {k: round(v[1], 3) for k, v in kdec.items()},
        "kernel_us_p8": {k: round(v[1], 3) for k, v in kp8.items()},
        "copy_kernel_gbs": copy_gbs,
        "decode_forward_us_by_context": sweep,
        "request_loops": full,
        "roofline": {
            "kernel": "proj_kernel<1,*,EPI_SILU> (gate|up + SiLU*up, decode row)",
            "bound": "hbm",
            "achieved": achieved,
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": achieved / HBM_PEAK_GBS,
            "traffic": traffic,
            "algorithmic_bytes_per_launch": gu_bytes,
            "avg_launch_us": gu_us,
        },
    }
    if not args.no_cpu_baseline:
        out["cpu_baseline"] = cpu_baseline(spec, synth, args.cpu_seconds)
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
