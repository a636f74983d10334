"""GPU parity of the hybrid (qwen35: gated full attention + gated delta net)
resident decode against the oracle's hybrid forward on identical seeded
weights: logits within 1e-3 relative L2 and an identical greedy argmax for 32
steps.  The reference has no CPU forward for this architecture, so the oracle
(pinned by the float64 restatement in test_oracle_hybrid.py) is the checker.
"""
import numpy as np
import pytest

import modelgen

pytestmark = pytest.mark.gpu
LOGIT_TOL = 1e-3


@pytest.fixture(scope="module")
def ctx(lrs):
    c = lrs.Context()
    yield c
    c.close()


def rel_l2(a, b):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / np.linalg.norm(b))


CASES = [
    ("hy-tiny", modelgen.HY_TINY, None),
    ("hy-mid", modelgen.HY_MID, None),
    ("hy-tiny-q8_0-attn", modelgen.HY_TINY,
     dict(attn_q=modelgen.Q8_0, attn_k=modelgen.Q8_0, attn_v=modelgen.Q8_0)),
]


@pytest.mark.parametrize("name,cfg,mix", CASES, ids=[c[0] for c in CASES])
def test_hybrid_decode_and_greedy_match_oracle(lrs, orc, ctx, name, cfg, mix):
    print(f"case {name}", flush=True)
    w = modelgen.hybrid_host_model(orc, cfg, seed=21, mix=mix)
    gm = modelgen.gpu_hybrid_model(lrs, ctx, cfg, w)
    om = orc.HybridModel(cfg, w, kv_f16=True, threads=8)
    rng = np.random.default_rng(7)
    prompt = rng.integers(0, cfg["vocab"], 12).tolist()
    worst = 0.0
    for pos, t in enumerate(prompt):
        g = gm.decode(t, pos)
        o = om.forward([t])
        worst = max(worst, rel_l2(g, o))
        assert rel_l2(g, o) < LOGIT_TOL, (pos, rel_l2(g, o))
        assert int(np.argmax(g)) == int(np.argmax(o)), pos
    assert len(gm) == len(prompt)
    print(f"{name}: worst rel L2 {worst:.2e}")
    # 32 greedy steps on the device == the oracle's greedy loop from a reset state
    gm.reset()
    om2 = orc.HybridModel(cfg, w, kv_f16=True, threads=8)
    want = modelgen.oracle_greedy(om2, prompt, 32)
    got = gm.generate_greedy(prompt, 32).tolist()
    assert got == want


def test_hybrid_batch_reset_and_position_rule(lrs, orc, ctx):
    cfg = modelgen.HY_TINY
    w = modelgen.hybrid_host_model(orc, cfg, seed=22)
    gm = modelgen.gpu_hybrid_model(lrs, ctx, cfg, w)
    assert gm.batch_size() == 1
    toks = [3, 1, 4, 1, 5, 9, 2, 6]
    for p, t in enumerate(toks):
        last = gm.decode(t, p)
    # the recurrent state cannot be rewound
    with pytest.raises(lrs.ModelError):
        gm.decode(toks[0], 3)
    gm.reset()
    b = gm.decode_batch(toks, 0)
    assert np.array_equal(b, last)  # same launches, same state after reset
    o = orc.HybridModel(cfg, w, kv_f16=True, threads=8).forward(toks)
    assert rel_l2(b, o) < LOGIT_TOL
    assert len(gm) == len(toks)
    # decode_batch continues the sequence
    nxt = gm.decode_batch([7, 8], len(toks))
    o2 = orc.HybridModel(cfg, w, kv_f16=True, threads=8)
    o2.forward(toks)
    assert rel_l2(nxt, o2.forward([7, 8])) < LOGIT_TOL


def test_hybrid_rejects_bad_shapes(lrs, orc, ctx):
    cfg = modelgen.HY_TINY
    w = modelgen.hybrid_host_model(orc, cfg, seed=23)
    with pytest.raises(lrs.ModelError):
        modelgen.gpu_hybrid_model(lrs, ctx, dict(cfg, dn_state=32), w)
    with pytest.raises(lrs.ModelError):
        modelgen.gpu_hybrid_model(lrs, ctx, dict(cfg, dn_k_heads=3), w)


def test_hybrid_profile_ops(lrs, orc, ctx):
    cfg = modelgen.HY_MID
    w = modelgen.hybrid_host_model(orc, cfg, seed=24)
    gm = modelgen.gpu_hybrid_model(lrs, ctx, cfg, w)
    gm.decode(1, 0)
    for op in ("dn_proj", "dn_step", "dn_out", "qkv", "qk_prep", "attn", "o", "gateup",
               "down", "head"):
        us, b = gm.profile(op, 4)
        assert us > 0 and b > 0, op
