"""GPU parity of the resident decode (GpuResidentDecode) against the CPU
oracle's Model::forward on identical seeded weights.

Bars: logits within 1e-3 relative L2 and an identical
greedy argmax for 32 steps.  The oracle keeps K/V in f16 like the GPU cache
(integration.rs:872-893 does the same); a second check compares against the
pure f32-cache reference."""
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
    ("tiny-q4km", modelgen.TINY, modelgen.Q4_K_M, 1),
    ("tiny-q8_0", modelgen.TINY, modelgen.ALL_Q8_0, 1),
    ("tiny-q5km", modelgen.TINY, modelgen.Q5_K_M, 1),
    ("gqa5-q4km", modelgen.GQA5, modelgen.Q4_K_M, 1),
    ("gqa5-q4km-baseline-dist", modelgen.GQA5, modelgen.Q4_K_M, 0),
]


@pytest.mark.parametrize("name,cfg,mix,mode", CASES, ids=[c[0] for c in CASES])
def test_decode_logits_and_greedy_match_oracle(lrs, orc, ctx, name, cfg, mix, mode):
    kw = dict(mode=mode) if mode == 1 else dict(mode=0, d_lo=1e-3, d_hi=1e-2)
    w = modelgen.host_model(orc, cfg, seed=11, mix=mix, **kw)
    gm = modelgen.gpu_model(lrs, ctx, cfg, w)
    om = orc.Model(cfg, w, kv_f16=True, threads=8)
    om32 = orc.Model(cfg, w, kv_f16=False, threads=8)
    rng = np.random.default_rng(5)
    prompt = rng.integers(0, cfg["vocab"], 12).tolist()
    worst = 0.0
    for pos, t in enumerate(prompt):
        g = gm.decode(t, pos)
        o = om.forward([t])
        o32 = om32.forward([t])
        worst = max(worst, rel_l2(g, o))
        assert rel_l2(g, o) < LOGIT_TOL, (pos, rel_l2(g, o))
        assert rel_l2(g, o32) < 10 * LOGIT_TOL, (pos, rel_l2(g, o32))
        assert int(np.argmax(g)) == int(np.argmax(o)), pos
    assert len(gm) == len(prompt)
    print(f"{name}: worst rel L2 {worst:.2e}")
    # 32 greedy steps on the device == the oracle's greedy loop
    gm.reset()
    om2 = orc.Model(cfg, w, kv_f16=True, threads=8)
    want = modelgen.oracle_greedy(om2, prompt, 32)
    got = gm.generate_greedy(prompt, 32).tolist()
    assert got == want


def test_decode_batch_equals_token_loop_and_reset_is_deterministic(lrs, orc, ctx):
    cfg = modelgen.TINY
    w = modelgen.host_model(orc, cfg, seed=12)
    gm = modelgen.gpu_model(lrs, ctx, cfg, w)
    toks = [3, 1, 4, 1, 5, 9, 2, 6]
    for p, t in enumerate(toks):
        last = gm.decode(t, p)
    gm.reset()
    b = gm.decode_batch(toks, 0)
    assert np.array_equal(b, last)
    assert gm.batch_size() >= 1 and len(gm) == len(toks)
    # greedy on device equals argmax of host logits
    gm.reset()
    gm.decode_batch(toks[:-1], 0)
    assert gm.decode_greedy(toks[-1], len(toks) - 1) == int(np.argmax(last))


def test_errors(lrs, orc, ctx):
    cfg = dict(modelgen.TINY, ctx=8)
    gm = modelgen.gpu_model(lrs, ctx, cfg, modelgen.host_model(orc, cfg, seed=13))
    with pytest.raises(lrs.ModelError) as e:
        gm.decode(1, 8)  # pos >= ctx: ContextOverflow
    assert e.value.code == -4
    with pytest.raises(lrs.ModelError):
        gm.decode(cfg["vocab"], 0)
    with pytest.raises(lrs.ModelError):
        gm.generate_greedy([1, 2, 3], 7)  # feeds positions 0..8 > ctx
    assert len(gm.generate_greedy([1, 2, 3], 6)) == 6  # the last token is not fed back
    gm.decode(1, 7)  # the last slot is fine


def test_model_rejects_bad_shapes(lrs, orc, ctx):
    from llama_rs_amd.model import ResidentForward

    cfg = modelgen.TINY
    w = modelgen.host_model(orc, cfg, seed=14)
    w["blk.1.ffn_up"] = w["blk.0.ffn_down"]  # wrong shape
    with pytest.raises(Exception):
        modelgen.gpu_model(lrs, ctx, cfg, w)
