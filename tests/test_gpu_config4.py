"""GPU parity at the hybrid benchmark's own width (the
27B-scale qwen35-shaped Q4_K_M model) cut to one block of four layers
(three gated delta-net layers, then one gated full-attention layer, as
full_attn_interval 4 puts them), against the CPU oracle's hybrid forward on
identical seeded weights.

Every decode kernel instance the config-4 benchmark times runs here at its
real shape: the delta-net projections (ssm_qkv 6144 + ssm_gate 2048 rows of
5120) with the fused RMSNorm, k_dn_step over 16 value heads of 128 x 128 f32
state (the gate dots over 5120 inputs, the causal conv of width 4, the gated
norm pack), ssm_out + residual, the gated attention's Q+gate (12288 rows) /
k / v projections, the QK-norm + partial RoPE (64 of 256 dims), the split
attention over 24 query / 4 KV heads x 256 with the sigmoid gate in the
combine, o + residual, gate/up + SwiGLU at n_ff 17408 and down; the prompt
block runs every full-width GEMM and the block delta-net kernels.  The
output head of 248320 Q6_K rows runs as a plain matvec.  The weights follow
the benchmark distributions (f16 scales uniform in [1e-3, 1e-2]).

Bars: logits within 1e-3 relative L2 of the oracle,
identical greedy tokens for 32 steps, the head matvec within 1e-4."""
import os

import numpy as np
import pytest

import modelgen

pytestmark = pytest.mark.gpu
LOGIT_TOL = 1e-3
THREADS = min(16, os.cpu_count() or 1)
C4_4L = dict(n_layer=4, n_embd=5120, n_head=24, n_head_kv=4, head_dim=256, n_ff=17408,
             vocab=4096, rope_dim=64, ctx=640, rms_eps=1e-6, freq_base=1e7,
             full_attn_interval=4, dn_k_heads=16, dn_v_heads=16, dn_state=128, dn_conv=4)


def rel_l2(a, b):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / np.linalg.norm(b))


@pytest.fixture(scope="module")
def c4(lrs, orc):
    ctx = lrs.Context(0)
    w, gm = modelgen.hybrid_device_model(lrs, ctx, orc, C4_4L, seed=41, mode=0, d_lo=1e-3,
                                         d_hi=1e-2)
    prompt = np.random.default_rng(19).integers(0, C4_4L["vocab"], 12).tolist()
    yield ctx, w, gm, prompt
    gm.close()
    ctx.close()


def test_config4_decode_logits_match_oracle(orc, c4):
    ctx, w, gm, prompt = c4
    gm.reset()
    om = orc.HybridModel(C4_4L, w, kv_f16=True, threads=THREADS)
    worst = 0.0
    for pos, t in enumerate(prompt):
        g = gm.decode(t, pos)
        o = om.forward([t])
        worst = max(worst, rel_l2(g, o))
        assert rel_l2(g, o) < LOGIT_TOL, (pos, rel_l2(g, o))
        assert int(np.argmax(g)) == int(np.argmax(o)), pos
    print(f"config-4 shape, 4 layers: worst rel L2 {worst:.2e} over {len(prompt)} steps")


def test_config4_greedy_32_steps_match_oracle(orc, c4):
    ctx, w, gm, prompt = c4
    gm.reset()
    om = orc.HybridModel(C4_4L, w, kv_f16=True, threads=THREADS)
    toks, margins = [], []
    logits = om.forward(np.asarray(prompt, np.uint32))
    for i in range(32):
        s = np.sort(logits)
        margins.append(float(s[-1] - s[-2]))
        toks.append(int(np.argmax(logits)))
        if i < 31:
            logits = om.forward([toks[-1]])
    got = gm.generate_greedy(prompt, 32).tolist()
    print(f"greedy top-1/top-2 margins: min {min(margins):.3f}, median {np.median(margins):.3f}")
    assert got == toks


def test_config4_prompt_block_matches_oracle(orc, c4):
    """decode_batch: the benchmark's 511-token prompt as one block (the
    full-width GEMMs, the block conv / gates / delta rule / gated norm, the
    batched QK-norm + RoPE and the causal attention at head_dim 256), then a
    decode step from the states and the cache the block leaves."""
    ctx, w, gm, _ = c4
    assert gm.batch_size() == 512
    gm.reset()
    toks = np.random.default_rng(29).integers(0, C4_4L["vocab"], 511).tolist()
    got = gm.decode_batch(toks, 0)
    om = orc.HybridModel(C4_4L, w, kv_f16=True, threads=THREADS)
    want = om.forward(np.asarray(toks, np.uint32))
    print(f"511-token block: rel L2 {rel_l2(got, want):.2e}")
    assert rel_l2(got, want) < LOGIT_TOL
    assert int(np.argmax(got)) == int(np.argmax(want))
    g = gm.decode(5, 511)
    o = om.forward([5])
    print(f"decode after the block: rel L2 {rel_l2(g, o):.2e}")
    assert rel_l2(g, o) < LOGIT_TOL
    assert int(np.argmax(g)) == int(np.argmax(o))


def test_config4_full_vocab_head_matvec(lrs, orc, c4):
    """the 248320-row Q6_K output head of config 4 (1.04 GB) within 1e-4"""
    ctx = c4[0]
    E, V = C4_4L["n_embd"], 248320
    W = lrs.Weight.generate(ctx, modelgen.Q6_K, 4141, E, V, mode=0, d_lo=1e-3, d_hi=1e-2)
    x = orc.gen_normal(98, E)
    got = W.matvec(x)
    ref = orc.matvec(modelgen.Q6_K, W.download(), E, V, x, threads=THREADS)
    W.free()
    print(f"head 248320 x 5120: rel L2 {rel_l2(got, ref):.2e}")
    assert rel_l2(got, ref) < 1e-4
