"""The decode's fused launches against their separate forms on the same
weights (the variables set to 0 at model creation):
- the attention combine in the o-projection's launch (k_mq_ao) against the
  combine kernel then the o matvec (LRS_AO=0);
- the hybrid's delta-net gate projections in the projection launch
  (k_mq_gates) against the step kernel computing them (LRS_DN_GATES=0).
- the split kernel's query heads split by one lane group each and shared
  through LDS against every lane group splitting every head (LRS_ATTN_DQ=0);
- the dense q/k/v epilogue's RoPE angles from the embed kernel's table
  against sincosf in the epilogue (LRS_ROPE_TABLE=0);
- the hybrid's QK-norm + RoPE in the attention split kernel against its own
  launch (LRS_QKP=0), within a tolerance (see below).
The first four run the same arithmetic in the same order (the combine's
merge, the pack, the matvec's units and K-slice sums; the gate dots'
per-thread sums, wavefront sums and their combination), so the logits must
be bit-identical:
token by token, over greedy chains, and at cache lengths where the position
splits of the attention first own one, two and three blocks.  The cases
cover every o weight type k_mq_ao has (Q4_K / Q5_K / Q6_K), head dims 64 /
128 / 256, the gated attention of the hybrid model, and the benchmark widths
(40 query heads over 5120 inputs; 24 x 256 over 6144; 16 value heads over
5120), so each instance of the fused launches that a benchmark runs is
here.  Their parity with the CPU oracle is the rest of the GPU suite, which
runs them by default."""
import numpy as np
import pytest

import modelgen

pytestmark = pytest.mark.gpu

# the config-3 attention and o shapes with a small FFN and vocabulary
C3W = dict(n_layer=2, n_embd=5120, n_head=40, n_head_kv=8, head_dim=128, n_ff=1024,
           vocab=1024, rope_dim=128, ctx=1400, rms_eps=1e-6, freq_base=1e6)
# the config-4 gated attention (24 / 4 heads x 256 over 5120) after one
# delta-net layer, small FFN and vocabulary
C4W = dict(n_layer=2, n_embd=5120, n_head=24, n_head_kv=4, head_dim=256, n_ff=1024,
           vocab=1024, rope_dim=64, ctx=64, rms_eps=1e-6, freq_base=1e7,
           full_attn_interval=2, dn_k_heads=16, dn_v_heads=16, dn_state=128, dn_conv=4)

DENSE = [
    ("tiny-q4km", modelgen.TINY, modelgen.Q4_K_M),
    ("tiny-q5km", modelgen.TINY, modelgen.Q5_K_M),
    ("gqa5-o-q6k", modelgen.GQA5, dict(modelgen.Q4_K_M, attn_output=modelgen.Q6_K)),
    ("c3-width", C3W, modelgen.Q4_K_M),
    ("hd256-rep8", modelgen.HD256R8, modelgen.Q4_K_M),
]


@pytest.fixture(scope="module")
def ctx(lrs):
    c = lrs.Context(0)
    yield c
    c.close()


SWITCHES = ("LRS_AO", "LRS_DN_GATES", "LRS_QKP", "LRS_ATTN_DQ", "LRS_ROPE_TABLE", "LRS_SAO")


def _pair(monkeypatch, make, off=("LRS_AO",)):
    """(fused, separate) models built by make(): the default, then with the
    variables `off` set to 0."""
    for v in SWITCHES:
        monkeypatch.delenv(v, raising=False)
    fused = make()
    for v in off:
        monkeypatch.setenv(v, "0")
    try:
        split = make()
    finally:
        for v in off:
            monkeypatch.delenv(v)
    return fused, split


@pytest.mark.parametrize("name,cfg,mix", DENSE, ids=[c[0] for c in DENSE])
def test_combine_in_o_launch_is_bit_identical(lrs, orc, ctx, monkeypatch, name, cfg, mix):
    w = modelgen.host_model(orc, cfg, seed=23, mix=mix, mode=0, d_lo=1e-3, d_hi=1e-2)
    fused, split = _pair(monkeypatch, lambda: modelgen.gpu_model(lrs, ctx, cfg, w))
    try:
        rng = np.random.default_rng(29)
        prompt = rng.integers(0, cfg["vocab"], 10).tolist()
        for pos, t in enumerate(prompt):
            a, b = fused.decode(t, pos), split.decode(t, pos)
            assert np.array_equal(a, b), (name, pos, float(np.max(np.abs(a - b))))
        fused.reset()
        split.reset()
        assert fused.generate_greedy(prompt, 16).tolist() == split.generate_greedy(prompt, 16).tolist()
    finally:
        fused.close()
        split.close()


@pytest.mark.parametrize("name,cfg,mix", DENSE, ids=[c[0] for c in DENSE])
def test_split_query_heads_shared_through_lds_is_bit_identical(lrs, orc, ctx, monkeypatch, name,
                                                               cfg, mix):
    """The split kernel's query heads split into f16 hi / lo pairs by one
    lane group each and shared through LDS (the default) against every lane
    group splitting every head (LRS_ATTN_DQ=0): the same per-head arithmetic
    over the same lanes, so the logits are bit-identical."""
    w = modelgen.host_model(orc, cfg, seed=31, mix=mix, mode=0, d_lo=1e-3, d_hi=1e-2)
    fused, split = _pair(monkeypatch, lambda: modelgen.gpu_model(lrs, ctx, cfg, w), ("LRS_ATTN_DQ",))
    try:
        toks = np.random.default_rng(33).integers(0, cfg["vocab"], 40).tolist()
        for pos, t in enumerate(toks):
            a, b = fused.decode(t, pos), split.decode(t, pos)
            assert np.array_equal(a, b), (name, pos, float(np.max(np.abs(a - b))))
    finally:
        fused.close()
        split.close()


@pytest.mark.parametrize("name,cfg,mix", DENSE, ids=[c[0] for c in DENSE])
def test_rope_table_in_qkv_epilogue_is_bit_identical(lrs, orc, ctx, monkeypatch, name, cfg, mix):
    """The q/k/v epilogue's RoPE cosines and sines from the table the embed
    kernel writes (the default) against sincosf in the epilogue
    (LRS_ROPE_TABLE=0): the same expression on the same operands, so the
    logits are bit-identical over 40 positions (angles up to 39 rad)."""
    w = modelgen.host_model(orc, cfg, seed=35, mix=mix, mode=0, d_lo=1e-3, d_hi=1e-2)
    fused, split = _pair(monkeypatch, lambda: modelgen.gpu_model(lrs, ctx, cfg, w),
                         ("LRS_ROPE_TABLE",))
    try:
        toks = np.random.default_rng(37).integers(0, cfg["vocab"], 40).tolist()
        for pos, t in enumerate(toks):
            a, b = fused.decode(t, pos), split.decode(t, pos)
            assert np.array_equal(a, b), (name, pos, float(np.max(np.abs(a - b))))
        fused.reset()
        split.reset()
        assert fused.generate_greedy(toks[:8], 16).tolist() == split.generate_greedy(toks[:8], 16).tolist()
    finally:
        fused.close()
        split.close()


def test_combine_in_o_launch_at_split_boundaries(lrs, orc, ctx, monkeypatch):
    """C3W (8 KV heads: 32 splits, blocks 512 positions apart): every decode
    step up to the cache length where the splits first own a third block,
    so the combine weighs 1..32 live splits, then splits of two and three
    blocks."""
    cfg = C3W
    w = modelgen.host_model(orc, cfg, seed=37, mode=0, d_lo=1e-3, d_hi=1e-2)
    fused, split = _pair(monkeypatch, lambda: modelgen.gpu_model(lrs, ctx, cfg, w))
    try:
        last = modelgen.split_block_checks(cfg["n_head_kv"])[-1]  # a cache length
        assert last <= cfg["ctx"]
        toks = np.random.default_rng(41).integers(0, cfg["vocab"], last).tolist()
        for pos in range(last):
            a, b = fused.decode(toks[pos], pos), split.decode(toks[pos], pos)
            assert np.array_equal(a, b), (pos, float(np.max(np.abs(a - b))))
    finally:
        fused.close()
        split.close()


def _pair_sao(monkeypatch, make):
    """(split in the o launch, split launch then combine + o) models built
    by make(): LRS_SAO=1, then LRS_SAO=0."""
    for v in SWITCHES:
        monkeypatch.delenv(v, raising=False)
    monkeypatch.setenv("LRS_SAO", "1")
    try:
        fused = make()
        monkeypatch.setenv("LRS_SAO", "0")
        split = make()
    finally:
        monkeypatch.delenv("LRS_SAO")
    return fused, split


SAO_CASES = [
    ("tiny-q4km", modelgen.TINY, modelgen.Q4_K_M, False),
    ("gqa5-q4km", modelgen.GQA5, modelgen.Q4_K_M, False),
    ("ksplit-rep8", modelgen.KSPLIT, modelgen.Q4_K_M, False),
    ("c3-width", C3W, modelgen.Q4_K_M, False),
    ("hd256-rep8", modelgen.HD256R8, modelgen.Q4_K_M, False),
    ("hy-tiny", modelgen.HY_TINY, None, True),
    ("hy-mid", modelgen.HY_MID, None, True),
    ("c4-width", C4W, None, True),
]


@pytest.mark.parametrize("name,cfg,mix,hybrid", SAO_CASES, ids=[c[0] for c in SAO_CASES])
def test_split_in_o_launch_is_bit_identical(lrs, orc, ctx, monkeypatch, name, cfg, mix, hybrid):
    """The attention split, the combine and the o-projection in one launch
    (k_mq_sao; the splits' partials reach the combine through agent-scope
    stores and per-head flags) against the split launch then the combine + o
    launch: the same arithmetic in the same order, so the logits are
    bit-identical token by token and over a greedy chain.  The cases are
    every head shape the launch is built for: 64 / 128 / 256 dims with 2, 5
    and 8 query heads per KV head, the dense model's shared query split and
    the hybrid's QK-norm + RoPE in the split, at the benchmark widths too."""
    if hybrid:
        w = modelgen.hybrid_host_model(orc, cfg, seed=61, mode=0, d_lo=1e-3, d_hi=1e-2)
        make = lambda: modelgen.gpu_hybrid_model(lrs, ctx, cfg, w)
    else:
        w = modelgen.host_model(orc, cfg, seed=61, mix=mix, mode=0, d_lo=1e-3, d_hi=1e-2)
        make = lambda: modelgen.gpu_model(lrs, ctx, cfg, w)
    fused, split = _pair_sao(monkeypatch, make)
    try:
        toks = np.random.default_rng(67).integers(0, cfg["vocab"], 24).tolist()
        for pos, t in enumerate(toks):
            a, b = fused.decode(t, pos), split.decode(t, pos)
            assert np.array_equal(a, b), (name, pos, float(np.max(np.abs(a - b))))
        fused.reset()
        split.reset()
        assert fused.generate_greedy(toks[:8], 16).tolist() == split.generate_greedy(toks[:8], 16).tolist()
    finally:
        fused.close()
        split.close()


def test_split_in_o_launch_at_split_boundaries(lrs, orc, ctx, monkeypatch):
    """C3W with the split in the o launch: every decode step up to the cache
    length where the splits first own a third block, so the combine waits
    for 1..32 live splits' flags, then for splits of two and three blocks."""
    cfg = C3W
    w = modelgen.host_model(orc, cfg, seed=71, mode=0, d_lo=1e-3, d_hi=1e-2)
    fused, split = _pair_sao(monkeypatch, lambda: modelgen.gpu_model(lrs, ctx, cfg, w))
    try:
        last = modelgen.split_block_checks(cfg["n_head_kv"])[-1]
        assert last <= cfg["ctx"]
        toks = np.random.default_rng(73).integers(0, cfg["vocab"], last).tolist()
        for pos in range(last):
            a, b = fused.decode(toks[pos], pos), split.decode(toks[pos], pos)
            assert np.array_equal(a, b), (pos, float(np.max(np.abs(a - b))))
    finally:
        fused.close()
        split.close()


HYBRID_OFF = {"ao": ("LRS_AO",), "gates": ("LRS_DN_GATES",), "both": ("LRS_AO", "LRS_DN_GATES")}


@pytest.mark.parametrize("off", sorted(HYBRID_OFF))
@pytest.mark.parametrize("name,cfg", [("hy-tiny", modelgen.HY_TINY), ("hy-mid", modelgen.HY_MID),
                                      ("c4-width", C4W)])
def test_hybrid_fused_launches_are_bit_identical(lrs, orc, ctx, monkeypatch, name, cfg, off):
    w = modelgen.hybrid_host_model(orc, cfg, seed=43, mode=0, d_lo=1e-3, d_hi=1e-2)
    fused, split = _pair(monkeypatch, lambda: modelgen.gpu_hybrid_model(lrs, ctx, cfg, w),
                         HYBRID_OFF[off])
    try:
        prompt = np.random.default_rng(47).integers(0, cfg["vocab"], 10).tolist()
        for pos, t in enumerate(prompt):
            a, b = fused.decode(t, pos), split.decode(t, pos)
            assert np.array_equal(a, b), (name, pos, float(np.max(np.abs(a - b))))
        fused.reset()
        split.reset()
        assert fused.generate_greedy(prompt, 16).tolist() == split.generate_greedy(prompt, 16).tolist()
    finally:
        fused.close()
        split.close()


def rel_l2(a, b):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / np.linalg.norm(b))


@pytest.mark.parametrize("splits", [0, 3], ids=["default-splits", "3-splits"])
@pytest.mark.parametrize("name,cfg", [("hy-tiny", modelgen.HY_TINY), ("hy-mid", modelgen.HY_MID),
                                      ("c4-width", C4W)])
def test_qk_prep_in_split_matches_its_launch(lrs, orc, ctx, monkeypatch, name, cfg, splits):
    """The split kernel normalises q and k with a lane-group sum of squares
    where the separate launch sums by wavefronts, so the two differ by float
    rounding (a k element can then round to the neighbouring f16): logits
    within 1e-5 relative L2 of each other at every position, the same
    greedy chain, and both within the GPU suite's 1e-3 of the oracle at the
    last position.  The split that owns the current position changes every
    16 positions; with the default split count the positions cover the
    first block of every split, with 3 splits (LRS_ATTN_SPLITS) 150
    positions cover three blocks of each, so the current row is built in a
    split's first, second and third block."""
    n = 150 if splits else 16 * modelgen.attn_splits(cfg["n_head_kv"]) + 8
    cfg = dict(cfg, ctx=max(cfg["ctx"], n + 24))
    w = modelgen.hybrid_host_model(orc, cfg, seed=53, mode=0, d_lo=1e-3, d_hi=1e-2)
    if splits:
        monkeypatch.setenv("LRS_ATTN_SPLITS", str(splits))
    fused, split = _pair(monkeypatch, lambda: modelgen.gpu_hybrid_model(lrs, ctx, cfg, w),
                         ("LRS_QKP",))
    try:
        seq = np.random.default_rng(59).integers(0, cfg["vocab"], n).tolist()
        worst = 0.0
        for pos, t in enumerate(seq):
            a, b = fused.decode(t, pos), split.decode(t, pos)
            e = rel_l2(a, b)
            worst = max(worst, e)
            assert e < 1e-5, (name, pos, e)
        om = orc.HybridModel(cfg, w, kv_f16=True, threads=8)
        o = om.forward(seq)
        assert rel_l2(a, o) < 1e-3 and rel_l2(b, o) < 1e-3, (rel_l2(a, o), rel_l2(b, o))
        fused.reset()
        split.reset()
        prompt = seq[:10]
        assert fused.generate_greedy(prompt, 16).tolist() == split.generate_greedy(prompt, 16).tolist()
        print(f"{name}: {n} positions, worst rel L2 {worst:.2e}")
    finally:
        fused.close()
        split.close()


def test_wait_bound_reports_an_error(lrs, orc, ctx, monkeypatch):
    """The o workgroups' wait for the combine's flags is bounded.  With
    LRS_AO_WAIT_TEST the combine workgroups raise no flags and every wait
    gives up after 16 polls (each kernel still ends), so decoding must fail
    with the library's HIP error instead of returning logits; a model made
    without the switch decodes normally."""
    cfg = modelgen.TINY
    w = modelgen.host_model(orc, cfg, seed=23, mode=0, d_lo=1e-3, d_hi=1e-2)
    monkeypatch.setenv("LRS_AO_WAIT_TEST", "1")
    try:
        bad = modelgen.gpu_model(lrs, ctx, cfg, w)
    finally:
        monkeypatch.delenv("LRS_AO_WAIT_TEST")
    try:
        for call in (lambda: bad.decode(1, 0), lambda: bad.generate_greedy([1, 2, 3], 4)):
            bad.reset()
            with pytest.raises(lrs.ModelError) as err:
                call()
            assert err.value.code == -2 and "ran out" in str(err.value), err.value
    finally:
        bad.close()
    good = modelgen.gpu_model(lrs, ctx, cfg, w)
    try:
        assert np.all(np.isfinite(good.decode(1, 0)))
    finally:
        good.close()
