"""bench.py — batch-1 quantized decode hot path on one MI355X.

Workloads:
  layer   config 2: one Qwen2.5-14B-shaped decoder layer matvec set (q,k,v,o,
          gate,up in Q4_K / v,down in Q6_K), batch 1, f32 activations.
          A step is one pass over the 7 matvecs; weights rotate over enough
          copies (> 2x the 256 MB Infinity Cache) that every byte comes from HBM.
Prints one JSON line (driver contract) with a roofline object for the dominant
kernel (Q4_K matvec) and the CPU oracle timed on a bounded sample.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

REPO = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, REPO)
sys.path.insert(0, os.path.join(REPO, "tests"))

HBM_PEAK_GBS = 8000.0
F32, F16, Q4_0, Q8_0, Q4_K, Q5_K, Q6_K = 0, 1, 2, 8, 12, 13, 14

CFG2 = [("attn_q", Q4_K, 5120, 5120), ("attn_k", Q4_K, 5120, 1024),
        ("attn_v", Q6_K, 5120, 1024), ("attn_output", Q4_K, 5120, 5120),
        ("ffn_gate", Q4_K, 5120, 13824), ("ffn_up", Q4_K, 5120, 13824),
        ("ffn_down", Q6_K, 13824, 5120)]
TS = {Q8_0: 34, Q4_K: 144, Q5_K: 176, Q6_K: 210}
BS = {Q8_0: 32, Q4_K: 256, Q5_K: 256, Q6_K: 256}


def gguf_bytes(t, n_in, n_out):
    return n_out * n_in // BS[t] * TS[t]


def log(msg):
    print(msg, file=sys.stderr, flush=True)


def bench_layer(lrs, ctx, steps, warmup):
    copies = 4  # 4 x 174.4 MB = 698 MB of distinct weights per rotation
    mats = []
    for c in range(copies):
        mats.append([lrs.Weight.generate(ctx, t, 100 * c + i, n_in, n_out)
                     for i, (_, t, n_in, n_out) in enumerate(CFG2)])
    set_bytes = sum(gguf_bytes(t, n_in, n_out) for _, t, n_in, n_out in CFG2)
    act_bytes = sum(4 * (n_in + n_out) for _, t, n_in, n_out in CFG2)
    xbuf = ctx.alloc(4 * 13824)
    ybuf = ctx.alloc(4 * 13824)
    xbuf.upload(np.random.default_rng(7).standard_normal(13824).astype(np.float32))

    def step(s):
        for w in mats[s % copies]:
            w.matvec_dev(xbuf, ybuf)

    for s in range(warmup):
        step(s)
    ctx.sync()
    ctx.timer_start()
    for s in range(steps):
        step(s)
    ms = ctx.timer_stop()
    per_set_ms = ms / steps

    # dominant kernel alone: Q4_K ffn_gate/up 13824x5120 over 16 rotating copies
    gates = [lrs.Weight.generate(ctx, Q4_K, 5000 + c, 5120, 13824) for c in range(16)]
    n_launch = 16 * 20
    for w in gates:
        w.matvec_dev(xbuf, ybuf)
    ctx.sync()
    ctx.timer_start()
    for i in range(n_launch):
        gates[i % 16].matvec_dev(xbuf, ybuf)
    k_ms = ctx.timer_stop() / n_launch
    k_bytes = gguf_bytes(Q4_K, 5120, 13824) + 4 * (5120 + 13824)
    return {
        "per_set_ms": per_set_ms,
        "set_bytes": set_bytes + act_bytes,
        "gbs": (set_bytes + act_bytes) / (per_set_ms * 1e-3) / 1e9,
        "kernel": "k_matvec<Q4_K> 13824x5120",
        "kernel_us": k_ms * 1e3,
        "kernel_bytes": k_bytes,
        "kernel_gbs": k_bytes / (k_ms * 1e-3) / 1e9,
    }


def cpu_baseline_layer():
    """Oracle (C restatement of dequant + sequential f32 dot) on the ffn_gate
    matrix, all host threads; scaled to GB/s of GGUF bytes."""
    import oracle

    threads = min(16, os.cpu_count() or 1)
    t, n_in, n_out = Q4_K, 5120, 13824
    w = oracle.gen_weight(t, 1, n_out, n_in)
    x = oracle.gen_normal(2, n_in)
    oracle.matvec(t, w, n_in, n_out, x, threads=threads)  # warm
    reps, t0 = 0, time.perf_counter()
    while time.perf_counter() - t0 < 10.0:
        oracle.matvec(t, w, n_in, n_out, x, threads=threads)
        reps += 1
    dt = (time.perf_counter() - t0) / reps
    b = gguf_bytes(t, n_in, n_out) + 4 * (n_in + n_out)
    return {"value": round(b / dt / 1e9, 3), "unit": "GB/s", "cores": threads, "kind": "port",
            "sample": f"{reps} x Q4_K ffn_gate 13824x5120 matvec (dequant + sequential f32 dot "
                      f"per row, rows in chunks of 32 over {threads} threads), ~10 s"}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--workload", default="layer", choices=["layer"])
    ap.add_argument("--no-cpu", action="store_true")
    a = ap.parse_args()
    if a.gpus != 1:
        print("bench.py measures one GPU: the decode path keeps the whole model resident on a "
              "single MI355X and nothing crosses GPUs (see DESIGN.md, 'Sharding').",
              file=sys.stderr)
        sys.exit(2)
    from pkgload import load_product

    lrs = load_product()
    ctx = lrs.Context()
    log(f"[bench] workload={a.workload} steps={a.steps} warmup={a.warmup}")
    r = bench_layer(lrs, ctx, a.steps, a.warmup)
    log(f"[bench] layer set {r['per_set_ms']*1e3:.1f} us ({r['gbs']:.0f} GB/s); "
        f"{r['kernel']} {r['kernel_us']:.2f} us ({r['kernel_gbs']:.0f} GB/s)")
    cpu = None if a.no_cpu else cpu_baseline_layer()
    out = {
        "metric": "quant matvec HBM GB/s, Qwen2.5-14B layer matvec set (batch-1 decode)",
        "value": round(r["gbs"], 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": a.steps,
        "warmup": a.warmup,
        "ms_per_step": round(r["per_set_ms"], 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32 (Q4_K/Q6_K weights)",
        "data": "synthetic (seeded GGUF blocks, BASELINE distributions)",
        "config": {"workload": "qwen2.5-14b-layer-matvec-set", "batch": 1, "n_embd": 5120,
                   "n_ff": 13824, "weights": "q,k,o,gate,up Q4_K; v,down Q6_K",
                   "copies_rotated": 4},
        "roofline": {"bound": "hbm", "achieved": round(r["kernel_gbs"], 1),
                     "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(r["kernel_gbs"] / HBM_PEAK_GBS, 4), "traffic": None,
                     "kernel": r["kernel"], "kernel_us": round(r["kernel_us"], 3)},
        "cpu_baseline": cpu,
    }
    print(json.dumps(out), flush=True)
    ctx.close()


if __name__ == "__main__":
    main()
