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
    c = lrs.Context(0)
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


def test_hybrid_long_context_decode_matches_oracle(lrs, orc, ctx):
    """The gated attention layers (6 query heads over one 256-dim KV head,
    k_attn<256, 6>) at the cache lengths where the position splits first own
    one, two and three 16-position blocks and one past each (computed from the
    split count, so a change of it moves the checks along); every token
    through decode(), checked at those lengths against the oracle."""
    checks = modelgen.split_block_checks(modelgen.HY_MID["n_head_kv"])
    cfg = dict(modelgen.HY_MID, ctx=max(checks) + 8)
    w = modelgen.hybrid_host_model(orc, cfg, seed=23)
    gm = modelgen.gpu_hybrid_model(lrs, ctx, cfg, w)
    om = orc.HybridModel(cfg, w, kv_f16=True, threads=8)
    seq = np.random.default_rng(13).integers(0, cfg["vocab"], max(checks)).tolist()
    done, worst = 0, 0.0
    for pos, t in enumerate(seq):
        g = gm.decode(t, pos)
        n = pos + 1
        if n in checks:
            o = om.forward(seq[done:n])
            done = n
            e = rel_l2(g, o)
            worst = max(worst, e)
            assert e < LOGIT_TOL, (n, e)
            assert int(np.argmax(g)) == int(np.argmax(o)), n
    gm.close()
    print(f"hy-mid long: worst rel L2 {worst:.2e} at lengths {checks}")


def test_hybrid_decode_fills_the_cache(lrs, orc, ctx):
    """Every position of a 64-position cache through decode() (the split
    kernel clamps its first block's loads into the cache and writes the
    current K/V row itself), checked against the oracle at the last
    positions and greedy-continued from a reset."""
    cfg = modelgen.HY_TINY
    w = modelgen.hybrid_host_model(orc, cfg, seed=29)
    gm = modelgen.gpu_hybrid_model(lrs, ctx, cfg, w)
    om = orc.HybridModel(cfg, w, kv_f16=True, threads=8)
    seq = np.random.default_rng(31).integers(0, cfg["vocab"], cfg["ctx"]).tolist()
    try:
        done = 0
        for pos, t in enumerate(seq):
            g = gm.decode(t, pos)
            if pos + 1 in (cfg["ctx"] - 1, cfg["ctx"]):
                o = om.forward(seq[done:pos + 1])
                done = pos + 1
                assert rel_l2(g, o) < LOGIT_TOL, (pos, rel_l2(g, o))
                assert int(np.argmax(g)) == int(np.argmax(o)), pos
        gm.reset()
        om2 = orc.HybridModel(cfg, w, kv_f16=True, threads=8)
        want = modelgen.oracle_greedy(om2, seq[:8], cfg["ctx"] - 8)
        assert gm.generate_greedy(seq[:8], cfg["ctx"] - 8).tolist() == want
    finally:
        gm.close()


def test_hybrid_batch_reset_and_position_rule(lrs, orc, ctx):
    """decode_batch runs the prompt block through the GEMMs, the block
    delta-net kernels and the batched gated attention; the token loop and the
    block agree with the oracle and with each other (argmax), and the state
    the block leaves (recurrent states, conv ring, KV) carries the decode on."""
    cfg = modelgen.HY_TINY
    w = modelgen.hybrid_host_model(orc, cfg, seed=22)
    gm = modelgen.gpu_hybrid_model(lrs, ctx, cfg, w)
    assert gm.batch_size() == 512
    toks = [3, 1, 4, 1, 5, 9, 2, 6]
    for p, t in enumerate(toks):
        last = gm.decode(t, p)
    # the recurrent state cannot be rewound
    with pytest.raises(lrs.ModelError):
        gm.decode(toks[0], 3)
    gm.reset()
    b = gm.decode_batch(toks, 0)
    om = orc.HybridModel(cfg, w, kv_f16=True, threads=8)
    o = om.forward(toks)
    assert rel_l2(b, o) < LOGIT_TOL and rel_l2(last, o) < LOGIT_TOL
    assert int(np.argmax(b)) == int(np.argmax(last)) == int(np.argmax(o))
    assert len(gm) == len(toks)
    # decode_batch / decode continue the sequence from the block's state
    nxt = gm.decode_batch([7, 8], len(toks))
    assert rel_l2(nxt, om.forward([7, 8])) < LOGIT_TOL
    for p, t in enumerate([11, 12, 13], start=len(toks) + 2):
        assert rel_l2(gm.decode(t, p), om.forward([t])) < LOGIT_TOL


@pytest.mark.parametrize("name,cfg", [("hy-tiny", modelgen.HY_TINY), ("hy-mid", modelgen.HY_MID),
                                      ("hy-gqa5-256", dict(modelgen.HY_MID, n_head=5)),
                                      ("hy-ksplit", modelgen.HY_KS)])
def test_hybrid_prompt_block_matches_oracle(lrs, orc, ctx, name, cfg):
    """A 40-token prompt in one block (ring wrap, state carried across
    tokens inside the block kernel), then decode steps.  5 query heads per KV
    head at head_dim 256 splits the group over two workgroups of 3 wavefronts
    in the prompt attention, one of them idle."""
    cfg = dict(cfg, ctx=64)
    w = modelgen.hybrid_host_model(orc, cfg, seed=25)
    gm = modelgen.gpu_hybrid_model(lrs, ctx, cfg, w)
    om = orc.HybridModel(cfg, w, kv_f16=True, threads=8)
    prompt = np.random.default_rng(9).integers(0, cfg["vocab"], 40).tolist()
    g = gm.decode_batch(prompt, 0)
    o = om.forward(prompt)
    assert rel_l2(g, o) < LOGIT_TOL, rel_l2(g, o)
    for p, t in enumerate([1, 2, 3, 4], start=40):
        g, o = gm.decode(t, p), om.forward([t])
        assert rel_l2(g, o) < LOGIT_TOL, (p, rel_l2(g, o))
        assert int(np.argmax(g)) == int(np.argmax(o))


def test_hybrid_rejects_bad_shapes(lrs, orc, ctx):
    cfg = modelgen.HY_TINY
    w = modelgen.hybrid_host_model(orc, cfg, seed=23)
    with pytest.raises(lrs.ModelError):
        modelgen.gpu_hybrid_model(lrs, ctx, dict(cfg, dn_state=32), w)
    with pytest.raises(lrs.ModelError):
        modelgen.gpu_hybrid_model(lrs, ctx, dict(cfg, dn_k_heads=3), w)


def test_hybrid_profile_ops(lrs, orc, ctx, monkeypatch):
    """Every op times and counts bytes.  With the split in a launch of its
    own (LRS_SAO=0), the QK-norm + RoPE runs inside the attention split by
    default (qk_prep then reports nothing of its own and attn counts its
    bytes) and in a launch of its own with LRS_QKP=0.  By default the o
    launch also runs the split: attn reports nothing of its own and o counts
    both ops' bytes."""
    cfg = modelgen.HY_MID
    w = modelgen.hybrid_host_model(orc, cfg, seed=24)
    attn_b, o_b = {}, {}
    for qkp, sao in (("1", "0"), ("0", "0"), ("1", "1")):
        monkeypatch.setenv("LRS_QKP", qkp)
        monkeypatch.setenv("LRS_SAO", sao)
        gm = modelgen.gpu_hybrid_model(lrs, ctx, cfg, w)
        try:
            gm.decode(1, 0)
            for op in ("dn_proj", "dn_step", "dn_out", "qkv", "qk_prep", "attn", "o", "gateup",
                       "down", "head"):
                us, b = gm.profile(op, 4)
                if (op == "qk_prep" and qkp == "1") or (op == "attn" and sao == "1"):
                    assert us == 0 and b == 0, (op, qkp, sao)
                else:
                    assert us > 0 and b > 0, (op, qkp, sao)
                if op == "attn":
                    attn_b[qkp + sao] = b
                if op == "o":
                    o_b[qkp + sao] = b
        finally:
            gm.close()
    kvd = cfg["n_head_kv"] * cfg["head_dim"]
    assert attn_b["10"] - attn_b["00"] == kvd * 12 + 3 * cfg["head_dim"] * 4
    assert o_b["11"] == o_b["10"] + attn_b["10"]
