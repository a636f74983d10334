"""bench.py — batch-1 quantized decode hot path on one MI355X.

Workloads:
  decode  config 3 (default): Qwen2.5-32B-shaped dense decoder, random-init
          Q4_K_M (q,k,o,gate,up Q4_K; v,down,output Q6_K; token_embd Q4_K),
          whole model resident on the GPU.  A 512-token prompt is consumed,
          then a step is one greedy decode token (one HIP-graph replay of the
          full forward, argmax on the device).  W warmup tokens are decoded
          at positions 511.., then the cache is rewound and K timed tokens are
          decoded at the same positions 511..511+K-1 (attention length
          512..511+K, the config's 128 tokens after a 512-token prompt).
  q8      config 1: one Q8_0 4096x4096 matvec (d ~ U[1e-3,1e-2], qs ~ U[-127,127],
          x ~ N(0,1) f32); a step is one lrs_matvec_dev call (one launch: each
          workgroup packs x, then the matrix-core matvec), 16 of them over 16 weight copies (285 MB, beyond
          the 256 MB MALL, so every weight byte comes from HBM) captured into
          one HIP graph and replayed.
  layer   config 2: one Qwen2.5-14B-shaped layer matvec set through the token
          plan's fused launches (q/k/v in one launch, o, gate/up + SwiGLU,
          down) of a 4-layer model of that shape, rotating over the layers so
          every byte comes from HBM; also, labelled, the same 7 matvecs as
          separate lrs_matvec_dev calls (one captured HIP graph per copy).
  hybrid  config 4: 27B-scale hybrid model (64 layers, gated full attention
          every 4th: 24 q / 4 kv x 256; 48 gated delta-net layers of 16 heads
          x 128x128 f32 state), random-init Q4_K_M; the 512-token prompt goes
          through one batched block (GEMMs + block delta-net kernels), then K
          greedy tokens are timed at positions 511..  (warmup runs on a separate
          pass: the recurrent state cannot be rewound, so the model is reset
          and the prompt replayed before the timed tokens).
  prefill config 5 through the full model: a prompt of M tokens (--m: 128 /
          512 / 2048) consumed by the 32B-shaped model of config 3 in blocks of
          512 tokens (bf16 hi/lo matrix-core GEMMs for every projection,
          batched norm / RoPE / causal attention); a step is one whole prompt.
          Reports prompt tok/s and the algorithmic matmul TFLOP/s (2 x M x
          weight elements; the hi/lo split issues three bf16 products each).
  pmc     profiling helper for the rocprofv3 counter passes: a plain copy
          kernel of known size (calibration) and the dominant decode kernel
          on a 4-layer model of the 32B shape.

One JSON line (driver contract) with a roofline object for the dominant
kernel, measured with HIP events on the model's stream, and the CPU oracle
(its -O3 -march=native timing build, compiled on the host that runs it)
timed on a bounded sample of the same workload.  The default decode line
also carries labelled lines for configs 1, 2, 4 and 5 under "configs"
(--no-sub skips them).
"""
from __future__ import annotations

import argparse
import json
import os
import re
import sys
import time

import numpy as np

REPO = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, REPO)
sys.path.insert(0, os.path.join(REPO, "tests"))

HBM_PEAK_GBS = 8000.0
METRIC = "batch-1 decode tok/s Q4_K_M 32B-shape; quant matvec HBM GB/s vs peak"
F32, F16, Q4_0, Q8_0, Q4_K, Q5_K, Q6_K = 0, 1, 2, 8, 12, 13, 14
TS = {Q8_0: 34, Q4_K: 144, Q5_K: 176, Q6_K: 210}
BS = {Q8_0: 32, Q4_K: 256, Q5_K: 256, Q6_K: 256}
OP_NAMES = {"qkv": "fused RMSNorm + q/k/v matvec + bias + RoPE + f16 KV append",
            "attn": "split-K GQA attention over the f16 KV cache (run in the o launch by default, then 0 here)",
            "o": "attention split + combine + attn_output matvec + residual add (one launch)",
            "gateup": "fused RMSNorm + ffn_gate/ffn_up Q4_K matvec + SwiGLU",
            "down": "ffn_down Q6_K matvec + residual add",
            "ffn": "the layer's FFN as the token plan runs it (gate/up + SwiGLU launch, then down + residual)",
            "head": "final RMSNorm + output head Q6_K matvec"}
PROMPT = 512


def gguf_bytes(t, n_in, n_out):
    return n_out * n_in // BS[t] * TS[t]


def log(msg):
    print(msg, file=sys.stderr, flush=True)


def cfg32(n_layer=None):
    from llama_rs_amd.model import QWEN25_32B

    c = dict(QWEN25_32B)
    if n_layer:
        c["n_layer"] = n_layer
    return c


def op_profile(m, n_layer):
    """Average duration of every fused op (HIP events on the model's stream;
    per-layer ops rotate over all layers so weights stream from HBM)."""
    ops = {}
    for op in ("qkv", "attn", "o", "gateup", "down", "ffn", "head"):
        iters = 2 * n_layer if op != "head" else 8
        us, b = m.profile(op, iters)
        mult = n_layer if op != "head" else 1
        ops[op] = dict(us=us, bytes=b, per_token_us=us * mult, gbs=b / us / 1e3 if us else 0.0)
    return ops


def read_traffic(op):
    """HBM bytes per launch of `op` from the committed rocprofv3 counter
    summary (FETCH_SIZE + WRITE_SIZE, each scaled by the copy-kernel
    calibration), or None when no summary covers it."""
    path = os.path.join(REPO, "profiles", "pmc_decode_q4km.md")
    try:
        txt = open(path).read()
    except OSError:
        return None
    mt = re.search(r"^traffic_bytes_per_launch\[%s\]\s*=\s*(\d+)" % re.escape(op), txt, re.M)
    return int(mt.group(1)) if mt else None


def bench_decode(lrs, ctx, steps, warmup, prefill_ms=()):
    from llama_rs_amd.model import synthetic_model

    cfg = cfg32()
    if PROMPT + max(steps, warmup) > cfg["ctx"]:
        raise SystemExit(f"--steps/--warmup must keep {PROMPT} + tokens within ctx {cfg['ctx']}")
    t0 = time.perf_counter()
    m = synthetic_model(ctx, cfg, seed=1, mode=0, d_lo=1e-3, d_hi=1e-2)
    ctx.sync()
    log(f"[bench] 32B-shape Q4_K_M model resident in {time.perf_counter() - t0:.1f} s, "
        f"{m.bytes_per_token / 1e9:.3f} GB of GGUF weights per token")
    rng = np.random.default_rng(1234)
    prompt = rng.integers(0, cfg["vocab"], PROMPT).astype(np.uint32)
    t0 = time.perf_counter()
    m.decode_batch(prompt[:-1], 0)
    log(f"[bench] prompt {PROMPT - 1} tokens in {time.perf_counter() - t0:.2f} s (first call)")
    # the same prompt again, buffers allocated: the batched-prompt rate
    # (logits of the last token copied back included)
    m.reset()
    t0 = time.perf_counter()
    m.decode_batch(prompt[:-1], 0)
    prefill_s = time.perf_counter() - t0
    log(f"[bench] prompt {PROMPT - 1} tokens in {prefill_s:.3f} s -> "
        f"{(PROMPT - 1) / prefill_s:.0f} tok/s (batch_size {m.batch_size()})")
    last = prompt[-1:]
    if warmup:
        m.generate_greedy(last, warmup, pos0=PROMPT - 1)
    ctx.sync()
    # timed: K greedy tokens at positions 511..511+K-1 (the warmup tokens'
    # cache entries are overwritten in order)
    ctx.timer_start()
    w0 = time.perf_counter()
    toks = m.generate_greedy(last, steps, pos0=PROMPT - 1)
    ctx.sync()
    wall = time.perf_counter() - w0
    ev_ms = ctx.timer_stop()
    ms_tok = wall * 1e3 / steps
    log(f"[bench] {steps} tokens: wall {wall * 1e3:.1f} ms, events {ev_ms:.1f} ms "
        f"-> {steps / wall:.1f} tok/s; first tokens {toks[:6].tolist()}")
    # per-token algorithmic bytes: GGUF weights + f16 K/V read at each length
    kvd = cfg["n_head_kv"] * cfg["head_dim"]
    kv_bytes = np.mean([L * kvd * 2 * 2 * cfg["n_layer"]
                        for L in range(PROMPT, PROMPT + steps)])
    tok_bytes = m.bytes_per_token + kv_bytes
    ops = op_profile(m, cfg["n_layer"])
    for k, v in ops.items():
        log(f"[bench]   {k:7s} {v['us']:8.2f} us/launch {v['gbs']:7.0f} GB/s  "
            f"{v['per_token_us'] / 1e3:.3f} ms/token")
    # config 5 through the same model: whole prompts of each length
    prefill = {m_tok: time_prompts(m, ctx, cfg, m_tok, 2, 1) for m_tok in prefill_ms}
    m.close()
    return dict(cfg=cfg, ms_tok=ms_tok, ev_ms_tok=ev_ms / steps, tok_bytes=tok_bytes,
                prefill_tok_s=(PROMPT - 1) / prefill_s,
                kv_bytes=kv_bytes, w_bytes=m.bytes_per_token, ops=ops, prefill=prefill)


HY_OPS = ("dn_proj", "dn_step", "dn_out", "qkv", "qk_prep", "attn", "o", "gateup", "down",
          "head")
OP_NAMES.update({"dn_proj": "fused RMSNorm + delta-net qkv/z Q4_K matvec + gate projections",
                 "dn_step": "delta-net step: conv, L2, delta rule, gated norm",
                 "dn_out": "delta-net ssm_out matvec + residual add",
                 "qk_prep": "QK-norm + RoPE + f16 KV append (gated attention layers; 0 when the "
                            "attention split does it, the default)"})


def bench_hybrid(lrs, ctx, steps, warmup):
    from llama_rs_amd.model import QWEN35_27B, synthetic_hybrid_model

    cfg = dict(QWEN35_27B)
    if PROMPT + steps > cfg["ctx"]:
        raise SystemExit(f"--steps must keep {PROMPT} + tokens within ctx {cfg['ctx']}")
    t0 = time.perf_counter()
    m = synthetic_hybrid_model(ctx, cfg, seed=1, mode=0, d_lo=1e-3, d_hi=1e-2)
    ctx.sync()
    log(f"[bench] 27B-scale hybrid Q4_K_M model resident in {time.perf_counter() - t0:.1f} s, "
        f"{m.bytes_per_token / 1e9:.3f} GB of weights per token")
    rng = np.random.default_rng(1234)
    prompt = rng.integers(0, cfg["vocab"], PROMPT).astype(np.uint32)
    m.decode_batch(prompt[:-1], 0)  # first call: allocates the prompt-block buffers
    if warmup:
        m.generate_greedy(prompt[-1:], warmup, pos0=PROMPT - 1)
    m.reset()
    ctx.sync()
    t0 = time.perf_counter()
    m.decode_batch(prompt[:-1], 0)
    prefill_s = time.perf_counter() - t0
    log(f"[bench] prompt {PROMPT - 1} tokens in {prefill_s:.3f} s -> "
        f"{(PROMPT - 1) / prefill_s:.0f} tok/s (batch_size {m.batch_size()})")
    ctx.sync()
    ctx.timer_start()
    w0 = time.perf_counter()
    toks = m.generate_greedy(prompt[-1:], steps, pos0=PROMPT - 1)
    ctx.sync()
    wall = time.perf_counter() - w0
    ev_ms = ctx.timer_stop()
    log(f"[bench] {steps} tokens: wall {wall * 1e3:.1f} ms, events {ev_ms:.1f} ms "
        f"-> {steps / wall:.1f} tok/s; first tokens {toks[:6].tolist()}")
    n_attn = sum((l + 1) % cfg["full_attn_interval"] == 0 for l in range(cfg["n_layer"]))
    n_dn = cfg["n_layer"] - n_attn
    kvd = cfg["n_head_kv"] * cfg["head_dim"]
    kv_bytes = np.mean([L * kvd * 2 * 2 * n_attn for L in range(PROMPT, PROMPT + steps)])
    D, nv = cfg["dn_state"], cfg["dn_v_heads"]
    cd = (2 * cfg["dn_k_heads"] + nv) * D
    rec_bytes = n_dn * (nv * D * D * 4 * 2 + cd * 4 * cfg["dn_conv"])
    tok_bytes = m.bytes_per_token + kv_bytes + rec_bytes
    ops = {}
    for op in HY_OPS:
        mult = n_dn if op.startswith("dn_") else n_attn if op in ("qkv", "qk_prep", "attn",
                                                                   "o") else \
            1 if op == "head" else cfg["n_layer"]
        us, b = m.profile(op, 2 * mult if op != "head" else 8)
        ops[op] = dict(us=us, bytes=b, per_token_us=us * mult, gbs=b / us / 1e3 if us else 0.0)
        log(f"[bench]   {op:8s} {us:8.2f} us/launch {ops[op]['gbs']:7.0f} GB/s  "
            f"{us * mult / 1e3:.3f} ms/token")
    m.close()
    return dict(cfg=cfg, ms_tok=wall * 1e3 / steps, tok_bytes=tok_bytes, kv_bytes=kv_bytes,
                rec_bytes=rec_bytes, w_bytes=m.bytes_per_token, ops=ops, prefill_s=prefill_s)


_TIMING = {}


def cpu_oracle():
    """The oracle module switched to its -O3 -march=native timing build,
    compiled once per process on this host (the parity build stays as it is
    on disk)."""
    import tempfile

    import oracle

    if "path" not in _TIMING:
        _TIMING["path"] = oracle.use_timing_build(tempfile.mkdtemp(prefix="lrs_oracle_"))
    return oracle


def host_info(threads):
    """nproc, the threads this process may run on, the CPU model and the NUMA
    layout of the host that times the CPU baseline."""
    info = {"nproc": os.cpu_count(), "threads_used": threads,
            "build": "gcc -O3 -march=native (the oracle sources, built on this host)"}
    try:
        info["affinity_cpus"] = len(os.sched_getaffinity(0))
    except OSError:
        pass
    try:
        with open("/proc/cpuinfo") as f:
            info["cpu_model"] = next((ln.split(":", 1)[1].strip() for ln in f
                                      if ln.startswith("model name")), None)
    except OSError:
        info["cpu_model"] = None
    nodes, base = {}, "/sys/devices/system/node"
    try:
        for d in sorted(os.listdir(base)):
            if d.startswith("node") and d[4:].isdigit():
                with open(os.path.join(base, d, "cpulist")) as f:
                    nodes[d] = f.read().strip()
    except OSError:
        pass
    info["numa_nodes"] = nodes
    return info


def timed_rate(fn, secs):
    """(calls, seconds per call) of fn over about `secs` seconds, after one
    untimed call."""
    fn()
    k, t0 = 0, time.perf_counter()
    while time.perf_counter() - t0 < secs:
        fn()
        k += 1
    return k, (time.perf_counter() - t0) / k


def cpu_baseline_layer(threads):
    """Config 2 on the host: the oracle's 7 matvecs of the 14B layer set
    (dequant + sequential f32 dot per row, rows in chunks of 32 over
    `threads`), each weight its own seeded matrix."""
    oracle = cpu_oracle()
    ws = [(t, oracle.gen_weight(t, 100 + i, n_out, n_in), n_in, n_out)
          for i, (t, n_in, n_out) in enumerate(CFG14_SET)]
    xs = {n: oracle.gen_normal(7, n) for n in (5120, 13824)}
    b = sum(gguf_bytes(t, n_in, n_out) + 4 * (n_in + n_out) for t, n_in, n_out in CFG14_SET)
    k, t = timed_rate(lambda: [oracle.matvec(tt, w, n_in, n_out, xs[n_in], threads=threads)
                               for tt, w, n_in, n_out in ws], 6.0)
    return {"value": round(b / t / 1e9, 2), "unit": "GB/s", "cores": threads, "kind": "port",
            "sample": f"oracle dequant + f32 dot over the 7 matvecs of the set, {k} sets "
                      f"({t * 1e3:.1f} ms each, {threads} threads)",
            "host": host_info(threads)}


def cpu_baseline_gemm(threads, m):
    """Config 5 on the host: the oracle's batched matvec (8 columns per pass,
    dequant + sequential f32 dot) for m tokens over 1/64 of the rows of each
    FFN weight, scaled to the whole set."""
    oracle = cpu_oracle()
    shapes = [(Q4_K, 5120, 13824), (Q4_K, 5120, 13824), (Q6_K, 13824, 5120)]
    part = [(t, oracle.gen_weight(t, 500 + i, n_out // 64, n_in), n_in, n_out // 64)
            for i, (t, n_in, n_out) in enumerate(shapes)]
    xs = {n: oracle.gen_normal(5, m * n).reshape(m, n) for n in (5120, 13824)}
    k, t = timed_rate(lambda: [oracle.matvec(tt, w, n_in, n_out, xs[n_in], threads=threads)
                               for tt, w, n_in, n_out in part], 6.0)
    flop = sum(2.0 * m * n_in * n_out for _, n_in, n_out in shapes)
    return {"value": round(flop / (64 * t) / 1e12, 5), "unit": "TFLOP/s", "cores": threads,
            "kind": "port",
            "sample": f"oracle batched matvec, {m} columns over 1/64 of the rows of gate/up/down, "
                      f"{k} passes ({t * 1e3:.1f} ms each, {threads} threads); whole set = 64x",
            "host": host_info(threads)}


def cpu_baseline_hybrid(threads):
    """The oracle's hybrid forward on a bounded sample of config 4: one block of
    4 layers of the full shape (3 delta-net + 1 gated attention) timed over
    repeated tokens, plus 1/16 of the Q6_K output head's rows; scaled to one
    token = 16 blocks + the whole head."""
    import modelgen
    from llama_rs_amd.model import QWEN35_27B

    oracle = cpu_oracle()
    lc = dict(QWEN35_27B, n_layer=4, vocab=256, ctx=1024)
    w = modelgen.hybrid_host_model(oracle, lc, seed=3, mode=0, d_lo=1e-3, d_hi=1e-2)
    om = oracle.HybridModel(lc, w, kv_f16=True, threads=threads)
    om.forward([1])
    n, t0 = 0, time.perf_counter()
    while time.perf_counter() - t0 < 8.0 and n < 500:
        om.forward([(n * 7 + 3) % 256])
        n += 1
    t_block = (time.perf_counter() - t0) / n
    om.close()
    rows = 248320 // 16
    hw = oracle.gen_weight(Q6_K, 5, rows, 5120)
    x = oracle.gen_normal(1, 5120)
    oracle.matvec(Q6_K, hw, 5120, rows, x, threads=threads)
    nh, t0 = 0, time.perf_counter()
    while time.perf_counter() - t0 < 4.0:
        oracle.matvec(Q6_K, hw, 5120, rows, x, threads=threads)
        nh += 1
    t_head = (time.perf_counter() - t0) / nh * 16
    s_tok = 16 * t_block + t_head
    return {"value": round(1.0 / s_tok, 4), "unit": "tok/s", "cores": threads, "kind": "port",
            "sample": f"oracle hybrid forward: {n} single-token passes through a 4-layer block "
                      f"(3 delta-net + 1 gated attention) of the config-4 shape "
                      f"({t_block * 1e3:.1f} ms each) + {nh} matvecs over 1/16 of the Q6_K "
                      f"output head; per token = 16 blocks + 16x the head slice "
                      f"= {s_tok:.2f} s", "host": host_info(threads)}


def cpu_baseline_q8(threads):
    """Config 1 on the host: the oracle's dequant + sequential f32 dot
    (weights.rs:95-124 + ops.rs:78-101, rows in chunks of 32 over `threads`)
    on the 4096x4096 Q8_0 matvec, and, as a second labelled row, the
    int8-activation path Model::forward takes for Q8_0 weights
    (matmul_q8_0_actq, ops.rs:704-724, 728-886; one thread, scalar)."""
    oracle = cpu_oracle()
    n = 4096
    w = oracle.gen_weight(Q8_0, 900, n, n)
    x = oracle.gen_normal(1, n)
    b = gguf_bytes(Q8_0, n, n) + 8 * n
    k1, t1 = timed_rate(lambda: oracle.matvec(Q8_0, w, n, n, x, threads=threads), 4.0)
    k2, t2 = timed_rate(lambda: oracle.matvec_q8_0_actq(w, n, n, x), 4.0)
    return {"value": round(b / t1 / 1e9, 2), "unit": "GB/s", "cores": threads, "kind": "port",
            "sample": f"oracle dequant + f32 dot, {k1} matvecs of Q8_0 4096x4096 "
                      f"({t1 * 1e3:.2f} ms each, {threads} threads); second row: the "
                      f"int8-activation matmul_q8_0_actq restatement, {k2} matvecs "
                      f"({t2 * 1e3:.2f} ms each)",
            "int8_activation": {"value": round(b / t2 / 1e9, 2), "unit": "GB/s", "cores": 1,
                                "kind": "port",
                                "note": "scalar single-thread restatement, not the reference's "
                                        "rayon + AVX2 8-row kernels (ops.rs:766-880)"},
            "host": host_info(threads)}


def cpu_baseline_decode(threads):
    """The oracle (C restatement of Model::forward: per-row dequant + sequential
    f32 dot, rows in chunks of 32 over `threads`) on a bounded sample of the
    32B-shaped workload: one decoder layer of the full shape timed over
    repeated tokens, plus 1/8 of the Q6_K output head's rows; scaled to one
    token = 64 layers + the whole head."""
    import modelgen

    oracle = cpu_oracle()
    lc = cfg32(1)
    lc.update(vocab=256, ctx=1024)
    w = modelgen.host_model(oracle, lc, seed=3, mode=0, d_lo=1e-3, d_hi=1e-2)
    om = oracle.Model(lc, w, kv_f16=True, threads=threads)
    om.forward_partial([1], 1)
    n, t0 = 0, time.perf_counter()
    while time.perf_counter() - t0 < 8.0 and n < 1000:
        om.forward_partial([(n * 7 + 3) % 256], 1)
        n += 1
    t_layer = (time.perf_counter() - t0) / n
    om.close()
    rows = 152064 // 8
    hw = oracle.gen_weight(Q6_K, 5, rows, 5120)
    x = oracle.gen_normal(1, 5120)
    oracle.matvec(Q6_K, hw, 5120, rows, x, threads=threads)
    nh, t0 = 0, time.perf_counter()
    while time.perf_counter() - t0 < 4.0:
        oracle.matvec(Q6_K, hw, 5120, rows, x, threads=threads)
        nh += 1
    t_head = (time.perf_counter() - t0) / nh * 8
    s_tok = 64 * t_layer + t_head
    return {"value": round(1.0 / s_tok, 4), "unit": "tok/s", "cores": threads, "kind": "port",
            "sample": f"oracle Model::forward restatement: {n} single-token passes through one "
                      f"32B-shape Q4_K_M layer ({t_layer * 1e3:.1f} ms each, positions 1..{n}) "
                      f"+ {nh} matvecs over 1/8 of the Q6_K output head; per token = 64 layers "
                      f"+ 8x the head slice = {s_tok:.2f} s", "host": host_info(threads)}


def graphs_wanted():
    """Graph replay unless LRS_GRAPH=0 or rocprofv3 kernel tracing / counter
    collection is on (the model library applies the same rule to its own
    per-token graphs)."""
    def on(v):
        v = os.environ.get(v, "")
        return v not in ("", "0") and v.lower() != "false"
    return os.environ.get("LRS_GRAPH", "") != "0" and not on("ROCPROF_KERNEL_TRACE") and \
        not on("ROCPROF_COUNTER_COLLECTION")


class GraphOrDirect:
    """The launches of fn captured into one HIP graph, or (graphs_wanted()
    false) issued directly on the context stream each time."""

    def __init__(self, ctx, fn):
        self.fn = fn
        self.g = None if not graphs_wanted() else ctx.capture(fn)

    def launch(self):
        if self.g is None:
            self.fn()
        else:
            self.g.launch()

    def close(self):
        if self.g is not None:
            self.g.close()


CFG14 = dict(n_layer=4, n_embd=5120, n_head=40, n_head_kv=8, head_dim=128, n_ff=13824,
             vocab=256, rope_dim=128, ctx=1024, rms_eps=1e-6, freq_base=1e6)
CFG14_SET = [(Q4_K, 5120, 5120), (Q4_K, 5120, 1024), (Q6_K, 5120, 1024), (Q4_K, 5120, 5120),
             (Q4_K, 5120, 13824), (Q4_K, 5120, 13824), (Q6_K, 13824, 5120)]


def layer14_model(ctx):
    """The config-2 model with the o-projection as a plain matvec launch: the
    decode runs the attention combine in the o launch (LRS_AO), which is not
    part of the layer's matvec set."""
    from llama_rs_amd.model import synthetic_model

    old = os.environ.get("LRS_AO")
    os.environ["LRS_AO"] = "0"
    try:
        return synthetic_model(ctx, CFG14, seed=2, mode=0, d_lo=1e-3, d_hi=1e-2)
    finally:
        if old is None:
            del os.environ["LRS_AO"]
        else:
            os.environ["LRS_AO"] = old


def bench_layer(lrs, ctx, steps, warmup):
    """Config 2 through the token plan's fused launches: a 4-layer model of the
    14B shape (4 x 174 MB of weights, beyond the 256 MB MALL); a step is one
    layer's q/k/v, o, gate/up and down launches (lrs_model_profile
    LRS_OP_MATVECS, rotating over the layers).  Also timed, as a labelled
    second figure: the 7 matvecs as separate lrs_matvec_dev calls."""
    cfg = CFG14
    m = layer14_model(ctx)
    m.decode_batch(np.arange(8, dtype=np.uint32), 0)  # a valid cache position
    nl = cfg["n_layer"]
    m.profile("matvecs", max(nl, warmup))
    us, b = m.profile("matvecs", max(steps, nl))
    op_us = {op: m.profile(op, 4 * nl)[0] for op in ("qkv", "o", "gateup", "down")}
    m.close()
    log(f"[bench] 14B layer matvec set through the fused launches: {us:.2f} us "
        f"({b / us / 1e3:.0f} GB/s); " + ", ".join(f"{k} {v:.2f}" for k, v in op_us.items()))

    copies = 4
    mats = [[lrs.Weight.generate(ctx, t, 100 * c + i, n_in, n_out)
             for i, (t, n_in, n_out) in enumerate(CFG14_SET)] for c in range(copies)]
    xbuf, ybuf = ctx.alloc(4 * 13824), ctx.alloc(4 * 13824)
    xbuf.upload(np.random.default_rng(7).standard_normal(13824).astype(np.float32))
    mats[0][-1].matvec_dev(xbuf, ybuf)  # sizes the context scratch outside the capture
    ctx.sync()
    graphs = [GraphOrDirect(ctx, lambda c=c: [w.matvec_dev(xbuf, ybuf) for w in mats[c]])
              for c in range(copies)]
    for s in range(warmup):
        graphs[s % copies].launch()
    ctx.sync()
    ctx.timer_start()
    for s in range(steps):
        graphs[s % copies].launch()
    us_sep = ctx.timer_stop() * 1e3 / steps
    for g in graphs:
        g.close()
    for ws in mats:
        for w in ws:
            w.free()
    log(f"[bench] the same set as 7 separate matvecs: {us_sep:.2f} us")
    return dict(us=us, bytes=b, gbs=b / us / 1e3, op_us=op_us, us_separate=us_sep, layers=nl)


def bench_q8(lrs, ctx, steps, warmup):
    """16 matvecs (one per weight copy) captured into one HIP graph; a step
    is one matvec, the graph replayed ceil(steps / 16) times."""
    n = 4096
    copies = 16
    ws = [lrs.Weight.generate(ctx, Q8_0, 900 + c, n, n, mode=0, d_lo=1e-3, d_hi=1e-2)
          for c in range(copies)]
    xbuf, ybuf = ctx.alloc(4 * n), ctx.alloc(4 * n)
    xbuf.upload(np.random.default_rng(1234).standard_normal(n).astype(np.float32))
    reps = max(1, (steps + copies - 1) // copies)

    def timed(mv):
        mv(ws[0])  # sizes the context scratch outside the capture
        ctx.sync()
        g = GraphOrDirect(ctx, lambda: [mv(w) for w in ws])
        for _ in range(max(1, warmup // copies)):
            g.launch()
        ctx.sync()
        ctx.timer_start()
        for _ in range(reps):
            g.launch()
        t = ctx.timer_stop() * 1e3 / (reps * copies)
        g.close()
        return t

    us = timed(lambda w: w.matvec_dev(xbuf, ybuf))
    # second labelled row: the int8-activation path of the reference's CPU
    # forward for Q8_0 weights (x rounded to Q8_0, then the same matvec)
    us_actq = timed(lambda w: w.matvec_actq_dev(xbuf, ybuf))
    log(f"[bench] q8_0 matvec {us:.2f} us; int8-activation (actq) variant {us_actq:.2f} us")
    b = gguf_bytes(Q8_0, n, n) + 4 * n + 4 * n
    return dict(us=us, us_actq=us_actq, bytes=b, gbs=b / us / 1e3, matvecs=reps * copies)


def bench_gemm(lrs, ctx, steps, warmup, m, precision):
    """Config 5: M tokens x 5120 activations against Q4_K gate/up 13824x5120 and
    Q6_K down 5120x13824 (the config-2 FFN), on the matrix cores."""
    shapes = [("ffn_gate", Q4_K, 5120, 13824), ("ffn_up", Q4_K, 5120, 13824),
              ("ffn_down", Q6_K, 13824, 5120)]
    ws = [lrs.Weight.generate(ctx, t, 500 + i, n_in, n_out) for i, (_, t, n_in, n_out) in
          enumerate(shapes)]
    rng = np.random.default_rng(5)
    a_big = ctx.alloc(4 * m * 13824)
    y_big = ctx.alloc(4 * m * 13824)
    a_big.upload(rng.standard_normal(m * 13824).astype(np.float32))
    per = {}
    for (name, t, n_in, n_out), w in zip(shapes, ws):
        for _ in range(warmup):
            w.gemm_dev(a_big, y_big, m, precision)
        ctx.sync()
        ctx.timer_start()
        for _ in range(steps):
            w.gemm_dev(a_big, y_big, m, precision)
        us = ctx.timer_stop() * 1e3 / steps
        flops = 2.0 * m * n_in * n_out
        per[name] = dict(us=us, tflops=flops / us / 1e6)
    tot_us = sum(v["us"] for v in per.values())
    tot_flop = sum(2.0 * m * n_in * n_out for _, _, n_in, n_out in shapes)
    return dict(per=per, us=tot_us, tflops=tot_flop / tot_us / 1e6, flop=tot_flop)


def bench_gemm_library(steps, warmup, m):
    """The vendor library's bf16 GEMM (torch.matmul on ROCm: hipBLASLt) at the
    config-5 FFN shapes, its weights already dequantized to bf16: what a plain
    bf16 GEMM of these shapes reaches on this part, as a reference for the
    dequant-GEMM (not the product path: 2 B per weight instead of GGUF blocks,
    no dequantization).  Each shape rotates over 4 weight copies, so every
    weight byte comes from HBM."""
    import torch

    dev = torch.device("cuda", 0)
    gen = torch.Generator(device=dev)
    gen.manual_seed(5)
    shapes = [("ffn_gate", 5120, 13824), ("ffn_up", 5120, 13824), ("ffn_down", 13824, 5120)]
    per = {}
    for name, n_in, n_out in shapes:
        a = torch.randn(m, n_in, device=dev, dtype=torch.bfloat16, generator=gen)
        ws = [torch.randn(n_out, n_in, device=dev, dtype=torch.bfloat16, generator=gen)
              for _ in range(4)]
        for i in range(max(1, warmup)):
            torch.matmul(a, ws[i % 4].t())
        torch.cuda.synchronize()
        t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        t0.record()
        for i in range(steps):
            torch.matmul(a, ws[i % 4].t())
        t1.record()
        torch.cuda.synchronize()
        us = t0.elapsed_time(t1) * 1e3 / steps
        per[name] = dict(us=round(us, 2), tflops=round(2.0 * m * n_in * n_out / us / 1e6, 1))
        log(f"[bench]   library bf16 {name:9s} {us:9.1f} us {per[name]['tflops']:8.1f} TFLOP/s")
        del a, ws
    tot_us = sum(v["us"] for v in per.values())
    tot_flop = sum(2.0 * m * n_in * n_out for _, n_in, n_out in shapes)
    return {"metric": "library bf16 GEMM TFLOP/s at the config-5 FFN shapes (reference, "
                      "weights pre-dequantized to bf16)",
            "value": round(tot_flop / tot_us / 1e6, 2), "unit": "TFLOP/s", "n_gpus": 1,
            "steps": steps, "warmup": warmup, "higher_is_better": True,
            "dtype": "bf16 operands, f32 accumulate", "data": "synthetic (bf16 ~ N(0,1))",
            "config": {"workload": "config5-ffn-shapes-library-bf16-gemm", "m": m,
                       "op_us": {k: v["us"] for k, v in per.items()},
                       "op_tflops": {k: v["tflops"] for k, v in per.items()},
                       "frac_of_bf16_peak": round(tot_flop / tot_us / 1e6 / 2500.0, 4)}}


def time_prompts(m, ctx, cfg, m_tok, steps, warmup):
    """Config 5 through the full 32B-shaped model: one step = an m_tok-token
    prompt at positions 0.. (decode_batch: logits of the last token)."""
    if not 1 <= m_tok < cfg["ctx"]:
        raise SystemExit(f"--m must be within 1..{cfg['ctx'] - 1}")
    rng = np.random.default_rng(4321)
    prompt = rng.integers(0, cfg["vocab"], m_tok).astype(np.uint32)
    for _ in range(max(1, warmup)):
        m.decode_batch(prompt, 0)  # the first call allocates the prompt-block buffers
    ctx.sync()
    ctx.timer_start()
    w0 = time.perf_counter()
    for _ in range(steps):
        m.decode_batch(prompt, 0)
    ctx.sync()
    wall = time.perf_counter() - w0
    ev_ms = ctx.timer_stop()
    E, F, qd = cfg["n_embd"], cfg["n_ff"], cfg["n_head"] * cfg["head_dim"]
    kvd = cfg["n_head_kv"] * cfg["head_dim"]
    per_tok = 2.0 * cfg["n_layer"] * (E * qd + 2 * E * kvd + qd * E + 3 * E * F)
    s_step = wall / steps
    log(f"[bench] prompt {m_tok} tokens: {s_step * 1e3:.1f} ms per prompt (events "
        f"{ev_ms / steps:.1f} ms) -> {m_tok / s_step:.0f} tok/s, batch_size {m.batch_size()}")
    return dict(s=s_step, tok_s=m_tok / s_step, flop=per_tok * m_tok, steps=steps,
                tflops=per_tok * m_tok / s_step / 1e12)


def bench_prefill(lrs, ctx, steps, warmup, m_tok):
    from llama_rs_amd.model import synthetic_model

    cfg = cfg32()
    m = synthetic_model(ctx, cfg, seed=1, mode=0, d_lo=1e-3, d_hi=1e-2)
    r = time_prompts(m, ctx, cfg, m_tok, steps, warmup)
    m.close()
    return r


def run_pmc(lrs, ctx):
    """Kernels for the counter passes: the copy calibration (an F32 tensor's
    identity dequant: 4 B read + 4 B written per element, grid-stride), then
    phases separated by a marker launch (the same identity dequant on 4096
    elements): the decode ops rotating over 4 layers of the 32B shape; the
    same on a 4-layer block of the config-4 hybrid shape; the config-1 Q8_0
    matvec; the config-2 layer ops on 4 layers of the 14B shape; the config-5
    GEMMs at m = 512."""
    from llama_rs_amd.model import QWEN35_27B, synthetic_hybrid_model, synthetic_model

    n = 128 << 20  # 512 MiB read + 512 MiB written
    src = lrs.Weight.upload(ctx, F32, np.zeros(n, np.float32), n, 1)
    dst = ctx.alloc(4 * n)
    for _ in range(3):
        src.dequant_dev(dst)
    ctx.sync()
    log(f"[pmc] copy calibration: {3} launches of {4 * n} B read + {4 * n} B written")
    msrc = lrs.Weight.upload(ctx, F32, np.zeros(4096, np.float32), 4096, 1)

    def marker(name):
        msrc.dequant_dev(dst)
        ctx.sync()
        log(f"[pmc] phase {name}")

    marker("dense32")
    m = synthetic_model(ctx, cfg32(4), seed=1, mode=0, d_lo=1e-3, d_hi=1e-2)
    # a 512-token cache, so attention reads the decode-time length
    m.decode_batch(np.arange(PROMPT, dtype=np.uint32) % cfg32(4)["vocab"], 0)
    for op in ("qkv", "attn", "o", "gateup", "down", "head"):
        us, b = m.profile(op, 8 if op != "head" else 2)
        log(f"[pmc] {op}: {us:.2f} us/launch, {b} algorithmic bytes")
    m.close()
    marker("hybrid27")
    # config 4: the same ops on a 4-layer block of the hybrid shape (3 delta-net
    # layers + 1 gated attention layer)
    hm = synthetic_hybrid_model(ctx, dict(QWEN35_27B, n_layer=4), seed=1, mode=0, d_lo=1e-3,
                                d_hi=1e-2)
    hm.decode_batch(np.arange(8, dtype=np.uint32), 0)
    for op in ("gateup", "down", "dn_proj", "dn_step", "dn_out", "head"):
        us, b = hm.profile(op, 6 if op != "head" else 2)
        log(f"[pmc] hybrid {op}: {us:.2f} us/launch, {b} algorithmic bytes")
    hm.close()
    marker("q8")
    # config 1: the Q8_0 4096x4096 matvec (activation pack + matvec), 4 copies
    ws = [lrs.Weight.generate(ctx, Q8_0, 900 + c, 4096, 4096, mode=0, d_lo=1e-3, d_hi=1e-2)
          for c in range(4)]
    xb, yb = ctx.alloc(4 * 4096), ctx.alloc(4 * 4096)
    xb.upload(np.random.default_rng(1234).standard_normal(4096).astype(np.float32))
    for i in range(8):
        ws[i % 4].matvec_dev(xb, yb)
    ctx.sync()
    log(f"[pmc] q8 matvec: {gguf_bytes(Q8_0, 4096, 4096) + 8 * 4096} algorithmic bytes")
    for w in ws:
        w.free()
    marker("layer14")
    lm = layer14_model(ctx)
    lm.decode_batch(np.arange(8, dtype=np.uint32), 0)
    for op in ("qkv", "o", "gateup", "down"):
        us, b = lm.profile(op, 8)
        log(f"[pmc] l14 {op}: {us:.2f} us/launch, {b} algorithmic bytes")
    lm.close()
    marker("gemm")
    # config 5: the FFN GEMMs at m = 512 (bf16 operands)
    mm = 512
    gw = [lrs.Weight.generate(ctx, t, 500 + i, n_in, n_out)
          for i, (t, n_in, n_out) in enumerate([(Q4_K, 5120, 13824), (Q6_K, 13824, 5120)])]
    ab, yb2 = ctx.alloc(4 * mm * 13824), ctx.alloc(4 * mm * 13824)
    ab.upload(np.random.default_rng(5).standard_normal(mm * 13824).astype(np.float32))
    for w in gw:
        for _ in range(2):
            w.gemm_dev(ab, yb2, mm, 1)
    ctx.sync()
    log("[pmc] gemm: Q4_K 13824x5120 and Q6_K 5120x13824 at m = 512, 2 launches each")
    marker("end")


DTYPE = "f32 in/out; activations as 22-bit block fixed point (3 int8 digits) on int8 MFMA"


def common(a, value, unit, ms, higher=True):
    return {"value": value, "unit": unit, "n_gpus": 1, "steps": a.steps, "warmup": a.warmup,
            "ms_per_step": ms, "higher_is_better": higher, "scaling": "weak",
            "vs_baseline": None}


def line_decode(lrs, ctx, a, threads, prefill_ms=()):
    r = bench_decode(lrs, ctx, a.steps, a.warmup, prefill_ms)
    ops = r["ops"]
    # the dominant single kernel ("ffn" is two launches, reported in op_us)
    dom = max((k for k in ops if k != "ffn"), key=lambda k: ops[k]["per_token_us"])
    d = ops[dom]
    cpu = None if a.no_cpu else cpu_baseline_decode(threads)
    eff_gbs = r["tok_bytes"] / (r["ms_tok"] * 1e-3) / 1e9
    cfg = r["cfg"]
    out = {"metric": METRIC, **common(a, round(1e3 / r["ms_tok"], 2), "tok/s", round(r["ms_tok"], 4)),
           "dtype": DTYPE,
           "data": "synthetic (random-init Q4_K_M GGUF blocks generated on the GPU, BASELINE "
                   "distributions; prompt token ids uniform random, seed 1234)",
           "config": {"workload": "config3-qwen2.5-32b-shape-q4_k_m-greedy-decode",
                      "prompt": PROMPT, "decode_tokens": a.steps, "n_layer": cfg["n_layer"],
                      "n_embd": cfg["n_embd"], "n_head": cfg["n_head"],
                      "n_head_kv": cfg["n_head_kv"], "n_ff": cfg["n_ff"], "vocab": cfg["vocab"],
                      "kv": "f16", "ctx": cfg["ctx"],
                      "weights": "q,k,o,gate,up,token_embd Q4_K; v,down,output Q6_K",
                      "bytes_per_token": int(r["tok_bytes"]),
                      "token_roofline_frac": round(eff_gbs / HBM_PEAK_GBS, 4),
                      "effective_gbs": round(eff_gbs, 1),
                      "prompt_tok_s": round(r["prefill_tok_s"], 1),
                      "op_us": {k: round(v["us"], 2) for k, v in ops.items()}},
           "roofline": {"bound": "hbm", "achieved": round(d["gbs"], 1), "peak": HBM_PEAK_GBS,
                        "unit": "GB/s", "frac": round(d["gbs"] / HBM_PEAK_GBS, 4),
                        "traffic": read_traffic(dom), "kernel": OP_NAMES[dom], "op": dom,
                        "kernel_us": round(d["us"], 3), "bytes_per_launch": d["bytes"]},
           "cpu_baseline": cpu}
    return out, r


def line_hybrid(lrs, ctx, a, threads):
    r = bench_hybrid(lrs, ctx, a.steps, a.warmup)
    ops = r["ops"]
    dom = max(ops, key=lambda k: ops[k]["per_token_us"])
    d = ops[dom]
    cpu = None if a.no_cpu else cpu_baseline_hybrid(threads)
    cfg = r["cfg"]
    eff_gbs = r["tok_bytes"] / (r["ms_tok"] * 1e-3) / 1e9
    return {"metric": "batch-1 decode tok/s, hybrid attention + gated delta-net 27B-scale "
                      "Q4_K_M (config 4)",
            **common(a, round(1e3 / r["ms_tok"], 2), "tok/s", round(r["ms_tok"], 4)),
            "dtype": DTYPE,
            "data": "synthetic (random-init Q4_K_M GGUF blocks generated on the GPU, "
                    "BASELINE distributions; f32 delta-net vectors seeded; prompt ids "
                    "uniform random, seed 1234)",
            "config": {"workload": "config4-hybrid-27b-scale-q4_k_m-greedy-decode",
                       "prompt": PROMPT, "decode_tokens": a.steps,
                       **{k: cfg[k] for k in ("n_layer", "n_embd", "n_head", "n_head_kv",
                                              "head_dim", "n_ff", "vocab",
                                              "full_attn_interval", "dn_k_heads",
                                              "dn_v_heads", "dn_state", "dn_conv",
                                              "rope_dim")},
                       "weights": "q,k,o,gate,up,ssm_qkv,ssm_gate,ssm_out,token_embd Q4_K; "
                                  "v,down,output Q6_K; alpha/beta/conv/norms f32",
                       "bytes_per_token": int(r["tok_bytes"]),
                       "token_roofline_frac": round(eff_gbs / HBM_PEAK_GBS, 4),
                       "effective_gbs": round(eff_gbs, 1),
                       "prompt_tok_s": round((PROMPT - 1) / r["prefill_s"], 1),
                       "op_us": {k: round(v["us"], 2) for k, v in ops.items()}},
            "roofline": {"bound": "hbm", "achieved": round(d["gbs"], 1),
                         "peak": HBM_PEAK_GBS, "unit": "GB/s",
                         "frac": round(d["gbs"] / HBM_PEAK_GBS, 4),
                         "traffic": read_traffic("hybrid_" + dom),
                         "kernel": OP_NAMES[dom], "op": dom, "kernel_us": round(d["us"], 3),
                         "bytes_per_launch": d["bytes"]},
            "cpu_baseline": cpu}


def line_q8(lrs, ctx, a, threads):
    r = bench_q8(lrs, ctx, a.steps, a.warmup)
    return {"metric": "quant matvec HBM GB/s, single Q8_0 4096x4096 matvec (batch-1)",
            **common(a, round(r["gbs"], 2), "GB/s", round(r["us"] / 1e3, 6)),
            "dtype": DTYPE,
            "data": "synthetic (seeded Q8_0 blocks, BASELINE distributions; x ~ N(0,1))",
            "config": {"workload": "config1-q8_0-matvec-4096", "batch": 1,
                       "copies_rotated": 16, "bytes_per_matvec": r["bytes"],
                       "us_per_matvec": round(r["us"], 3),
                       "us_per_matvec_int8_activation": round(r["us_actq"], 3)},
            "roofline": {"bound": "hbm", "achieved": round(r["gbs"], 1),
                         "peak": HBM_PEAK_GBS, "unit": "GB/s",
                         "frac": round(r["gbs"] / HBM_PEAK_GBS, 4),
                         "traffic": read_traffic("q8_matvec"),
                         "kernel": "lrs_matvec_dev: Q8_0 matrix-core matvec, each workgroup "
                                   "packing the f32 input itself (one launch)",
                         "op": "q8_matvec", "kernel_us": round(r["us"], 3),
                         "bytes_per_launch": r["bytes"]},
            "cpu_baseline": None if a.no_cpu else cpu_baseline_q8(threads)}


def line_layer(lrs, ctx, a, threads):
    r = bench_layer(lrs, ctx, a.steps, a.warmup)
    tr = [read_traffic("l14_" + op) for op in ("qkv", "o", "gateup", "down")]
    return {"metric": "quant matvec HBM GB/s, Qwen2.5-14B layer matvec set (batch-1 decode)",
            **common(a, round(r["gbs"], 2), "GB/s", round(r["us"] / 1e3, 5)),
            "dtype": DTYPE,
            "data": "synthetic (random-init Q4_K_M GGUF blocks generated on the GPU, BASELINE "
                    "distributions)",
            "config": {"workload": "config2-qwen2.5-14b-layer-matvec-set", "batch": 1,
                       "layers_rotated": r["layers"], "bytes_per_set": r["bytes"],
                       "us_per_set": round(r["us"], 3),
                       "op_us": {k: round(v, 2) for k, v in r["op_us"].items()},
                       "us_per_set_as_7_separate_matvecs": round(r["us_separate"], 3)},
            "roofline": {"bound": "hbm", "achieved": round(r["gbs"], 1),
                         "peak": HBM_PEAK_GBS, "unit": "GB/s",
                         "frac": round(r["gbs"] / HBM_PEAK_GBS, 4),
                         "traffic": sum(tr) if all(t is not None for t in tr) else None,
                         "kernel": "the layer's matvec launches of the token plan: q/k/v (one "
                                   "launch), o, gate/up + SwiGLU, down",
                         "op": "matvecs", "kernel_us": round(r["us"], 3),
                         "bytes_per_launch": r["bytes"]},
            "cpu_baseline": None if a.no_cpu else cpu_baseline_layer(threads)}


def line_gemm(lrs, ctx, a, threads, m, precision):
    r = bench_gemm(lrs, ctx, a.steps, a.warmup, m, precision)
    for k, v in r["per"].items():
        log(f"[bench]   {k:9s} {v['us']:9.1f} us {v['tflops']:8.1f} TFLOP/s")
    peak = 2500.0  # MI355X dense bf16 MFMA
    return {"metric": "prefill dequant-GEMM TFLOP/s (config 5 FFN set, MFMA)",
            **common(a, round(r["tflops"], 2), "TFLOP/s", round(r["us"] / 1e3, 5)),
            "dtype": "bf16 operands, f32 accumulate" if precision == 1 else
                     "bf16 hi/lo split operands (3 products), f32 accumulate",
            "data": "synthetic (seeded GGUF blocks, x ~ N(0,1))",
            "config": {"workload": "config5-prefill-gemm-ffn", "m": m,
                       "weights": "gate/up Q4_K 13824x5120, down Q6_K 5120x13824",
                       "flop_per_step": r["flop"],
                       "op_us": {k: round(v["us"], 2) for k, v in r["per"].items()}},
            "roofline": {"bound": "mfma", "achieved": round(r["tflops"], 1), "peak": peak,
                         "unit": "TFLOP/s", "frac": round(r["tflops"] / peak, 4),
                         "traffic": read_traffic("gemm_set") if (m, precision) == (512, 1)
                         else None},
            "cpu_baseline": None if a.no_cpu else cpu_baseline_gemm(threads, m)}


def prefill_line(a, m_tok, r):
    peak = 2500.0  # MI355X dense bf16 MFMA
    return {"metric": "prefill tok/s through the 32B-shaped Q4_K_M model (config 5)",
            **common(a, round(r["tok_s"], 1), "tok/s", round(r["s"] * 1e3, 3)),
            "dtype": "bf16 hi/lo split operands (3 products), f32 accumulate",
            "data": "synthetic (random-init Q4_K_M GGUF blocks generated on the GPU; "
                    "prompt ids uniform random, seed 4321)",
            "config": {"workload": "config5-prefill-32b-model", "m": m_tok,
                       "block": 512, "matmul_flop_per_prompt": r["flop"]},
            "roofline": {"bound": "mfma", "achieved": round(r["tflops"], 1), "peak": peak,
                         "unit": "TFLOP/s", "frac": round(r["tflops"] / peak, 4),
                         "traffic": None, "mfma_work_per_flop": 3}}


STREAM_SIZES = {  # algorithmic bytes of the decode launches (config 3, then configs 1, 2, 4)
    "o": 14807040, "qkv": 22089728, "down": 116273152, "gateup": 159404032, "head": 639318016,
    "q8_matvec": 17858560, "l14_gateup": 79722496, "l14_down": 58157056,
    "hybrid_gateup": 100380672, "hybrid_down": 73224192}


def _probe_lib():
    """liblrs_probe.so: the load-only read kernel (a measurement library built
    beside liblrs.so, not part of the product)."""
    import ctypes as C

    path = os.path.join(REPO, "llama.rs_amd", "liblrs_probe.so")
    if not os.path.exists(path):
        raise SystemExit(f"{path} is missing: build first (python __graft_entry__.py)")
    L = C.CDLL(path)
    L.lrsp_read_time.restype = C.c_int
    L.lrsp_read_time.argtypes = [C.c_int, C.c_void_p, C.c_size_t, C.c_uint32, C.c_int,
                                 C.c_uint32, C.c_uint32, C.c_uint32, C.c_int,
                                 C.POINTER(C.c_float)]

    def read_time(device, ptr, window, n_windows, nt, workgroups=0, threads=0, reads=1,
                  plain_first=False):
        us = C.c_float()
        rc = L.lrsp_read_time(device, ptr, window, n_windows, 1 if nt else 0, workgroups,
                              threads, reads, 1 if plain_first else 0, C.byref(us))
        if rc != 0:
            raise RuntimeError(f"lrsp_read_time failed ({rc})")
        return us.value

    return read_time


def bench_stream(ctx, steps):
    """The read rate of a kernel that does nothing but stream
    (liblrs_probe.so), at each decode launch's byte count, best over
    512 / 1024 / 2048 workgroups: windows of that size step through a 1 GiB
    arena, so no window is still in the memory-side cache when it is read
    again (as in decode, which streams ~20 GB per token)."""
    read_time = _probe_lib()
    arena = 1 << 30
    buf = ctx.alloc(arena)
    dev = ctx.device
    out = {}
    for name, size in STREAM_SIZES.items():
        size -= size % 16
        nwin = max(1, arena // size)
        res = {}
        for nt in (True, False):
            per = {wg: read_time(dev, buf.ptr, size, nwin, nt, wg, 0, steps) for wg in (512, 1024, 2048)}
            wg = min(per, key=per.get)
            res["nt" if nt else "plain"] = dict(us=round(per[wg], 2), workgroups=wg,
                                                gbs=round(size / per[wg] / 1e3, 1))
        # the same window read once with plain loads just before (memory-side
        # cache warm), at the best non-temporal workgroup count
        wg = res["nt"]["workgroups"]
        us = read_time(dev, buf.ptr, size, nwin, True, wg, 0, min(steps, 8), plain_first=True)
        res["nt_after_plain"] = dict(us=round(us, 2), workgroups=wg, gbs=round(size / us / 1e3, 1))
        out[name] = dict(bytes=size, **res)
        log(f"[bench] stream {name:7s} {size / 1e6:7.1f} MB: nt {res['nt']['us']:7.2f} us "
            f"({res['nt']['gbs']:6.0f} GB/s, {res['nt']['workgroups']} workgroups), plain "
            f"{res['plain']['us']:7.2f} us, nt after a plain read {us:7.2f} us "
            f"({res['nt_after_plain']['gbs']:6.0f} GB/s)")
    # the read rate of 160 workgroups (one per CU on 160 of the 256 CUs, as
    # the decode down and o launches use) against 256, at down's size
    size = STREAM_SIZES["down"] - STREAM_SIZES["down"] % 16
    nwin = max(1, arena // size)
    cap = {}
    for wg, th in ((160, 256), (160, 768), (160, 1024), (256, 768), (256, 1024)):
        us = read_time(dev, buf.ptr, size, nwin, True, wg, th, steps)
        cap[f"{wg}x{th}"] = dict(us=round(us, 2), gbs=round(size / us / 1e3, 1),
                                 gbs_per_workgroup=round(size / us / 1e3 / wg, 1))
        log(f"[bench] stream down-size, {wg} workgroups x {th} threads: {us:7.2f} us "
            f"({size / us / 1e3:6.0f} GB/s, {size / us / 1e3 / wg:5.1f} per workgroup)")
    out["down_by_workgroups"] = cap
    buf.free()
    return out


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=128)
    ap.add_argument("--warmup", type=int, default=8)
    ap.add_argument("--workload", default="decode",
                    choices=["decode", "hybrid", "q8", "layer", "gemm", "gemm_library", "prefill",
                             "pmc", "stream"])
    ap.add_argument("--m", type=int, default=512,
                    help="gemm / prefill: prompt tokens (config 5: 128/512/2048)")
    ap.add_argument("--precision", type=int, default=1, choices=[1, 3],
                    help="gemm: 1 = bf16 operands, 3 = bf16 hi/lo split")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baselines")
    ap.add_argument("--no-sub", action="store_true",
                    help="decode: skip the labelled lines of configs 1, 2, 4 and 5")
    a = ap.parse_args()
    if a.gpus != 1:
        print(f"bench.py measures one GPU only (asked for {a.gpus}): the decode path keeps the "
              "whole model resident on a single MI355X and nothing crosses GPUs.",
              file=sys.stderr)
        sys.exit(2)
    if a.steps < 1:
        raise SystemExit("--steps must be >= 1")
    if a.workload == "gemm_library":
        # torch's own HIP runtime in a process that has not loaded this
        # library's (two HIP runtimes in one process see no device)
        print(json.dumps(bench_gemm_library(a.steps, a.warmup, a.m)), flush=True)
        return
    from pkgload import load_product

    lrs = load_product()
    ctx = lrs.Context(0)
    log(f"[bench] workload={a.workload} steps={a.steps} warmup={a.warmup}")
    threads = min(16, os.cpu_count() or 1)
    if a.workload == "pmc":
        run_pmc(lrs, ctx)
    elif a.workload == "stream":
        r = bench_stream(ctx, a.steps)
        print(json.dumps({"metric": "streaming read rate of a load-only kernel (liblrs_probe.so)",
                          "unit": "GB/s", "n_gpus": 1, "steps": a.steps, "data": "uninitialised "
                          "device memory (the values are not used)", "sizes": r}), flush=True)
    elif a.workload == "gemm":
        print(json.dumps(line_gemm(lrs, ctx, a, threads, a.m, a.precision)), flush=True)
    elif a.workload == "prefill":
        r = bench_prefill(lrs, ctx, a.steps, a.warmup, a.m)
        print(json.dumps(prefill_line(a, a.m, r)), flush=True)
    elif a.workload == "q8":
        print(json.dumps(line_q8(lrs, ctx, a, threads)), flush=True)
    elif a.workload == "layer":
        print(json.dumps(line_layer(lrs, ctx, a, threads)), flush=True)
    elif a.workload == "hybrid":
        print(json.dumps(line_hybrid(lrs, ctx, a, threads)), flush=True)
    else:
        sub = not a.no_sub
        out, r = line_decode(lrs, ctx, a, threads, prefill_ms=(128, 512, 2048) if sub else ())
        if sub:
            # the other BASELINE configs, each with its own roofline and CPU baseline
            sa = argparse.Namespace(**vars(a))
            sa.steps, sa.warmup = min(a.steps, 64), min(a.warmup, 8)
            out["configs"] = {
                "config1": line_q8(lrs, ctx, sa, threads),
                "config2": line_layer(lrs, ctx, sa, threads),
                "config4": line_hybrid(lrs, ctx, a, threads),
                "config5_gemm": line_gemm(lrs, ctx, argparse.Namespace(**dict(
                    vars(a), steps=10, warmup=2)), threads, 512, 1),
                "config5_prefill": {str(m): prefill_line(argparse.Namespace(**dict(
                    vars(a), steps=p["steps"], warmup=1)), m, p)
                    for m, p in r["prefill"].items()},
            }
        print(json.dumps(out), flush=True)
    ctx.close()


if __name__ == "__main__":
    main()
