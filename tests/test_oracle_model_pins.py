"""Pins the oracle's assembled forwards (lrso_model_forward, model.rs:99-266,
and lrso_hybrid_forward) with reductions the mathematics fixes, computed
here in float64 from the dequantized weights (dequant itself is pinned by
the reference's known answers and the gguf-py block):

* zeroed attn_output / ffn_down (or ssm_out) make every layer the identity,
  so the logits are the head applied to the normalised embedding;
* with one cached position the softmax has a single weight of exactly 1, so
  attention returns v (per GQA group) and q / k cannot change a single bit;
* with W_v = 0 every cached value row is the bias, so attention returns the
  bias at every position whatever the scores;
* with attn_output = 0 the layer is embedding + SwiGLU FFN in closed form;
* the gated delta rule from a zero state: after one token S = beta v k^T, so
  o = beta (k.q) v / sqrt(d); after two tokens the expansion of the rule
  gives o2 = (e^g2 beta1 (k1.q2) v1 + beta2 (k2.q2)(v2 - e^g2 beta1 (k1.k2) v1)) / sqrt(d),
  with the causal conv of the second token w[-2] x1 + w[-1] x2;
* Q8_0 weights go through the reference forward's int8-activation path
  (weights.rs:113-117) bit for bit.

Each reduction fails for a plausible mistake in the forward: residual
replaced instead of added, wrong norm weight, head on the wrong token, GQA
head mapping, unnormalised softmax, swapped gate / up, state transposed,
decay not applied or applied as g, sign of the delta correction, conv taps
reversed or shifted the wrong way, key head chosen by division instead of
modulo."""
import numpy as np
import pytest

import modelgen

F32, Q8_0, Q4_K, Q6_K = 0, 8, 12, 14
TOL = 1e-5


def rel(a, b):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / np.linalg.norm(b))


def deq(orc, w, name, n_in, n_out):
    t, arr = w[name]
    return orc.dequant(t, arr).astype(np.float64).reshape(n_out, n_in)


def rms(x, wv, eps):
    x = np.asarray(x, np.float64)
    return x / np.sqrt(np.mean(x * x) + eps) * np.asarray(wv, np.float64)


def silu(x):
    return x / (1.0 + np.exp(-x))


def embed(orc, cfg, w, tok):
    t, arr = w["token_embd"]
    rb = cfg["n_embd"] // orc.BLOCK[t] * orc.TYPE_SIZE[t]
    return orc.dequant(t, arr[tok * rb:(tok + 1) * rb]).astype(np.float64)


def head(orc, cfg, w, x):
    Wo = deq(orc, w, "output", cfg["n_embd"], cfg["vocab"])
    return Wo @ rms(x, w["output_norm"][1], cfg["rms_eps"])


def zero_like(orc, w, name):
    t, arr = w[name]
    return (t, np.zeros_like(arr))


CFG = dict(modelgen.TINY, n_layer=2, ctx=16)


# --------------------------------------------------------------------------
# dense forward
# --------------------------------------------------------------------------
def test_zero_mixer_and_ffn_give_embedding_then_head(orc):
    w = modelgen.host_model(orc, CFG, seed=21)
    for l in range(CFG["n_layer"]):
        for n in ("attn_output", "ffn_down"):
            w[f"blk.{l}.{n}"] = zero_like(orc, w, f"blk.{l}.{n}")
    m = orc.Model(CFG, w)
    for tok in (3, 400, 77, 3):
        got = m.forward([tok])
        assert rel(got, head(orc, CFG, w, embed(orc, CFG, w, tok))) < TOL


def _layer0_v_path(orc, cfg, w, e):
    """attention output of layer 0 for a single cached position: v of each
    query head's KV head (h // n_rep)"""
    E, H, HKV, HD = cfg["n_embd"], cfg["n_head"], cfg["n_head_kv"], cfg["head_dim"]
    h = rms(e, w["blk.0.attn_norm"][1], cfg["rms_eps"])
    v = deq(orc, w, "blk.0.attn_v", E, HKV * HD) @ h + w["blk.0.bv"][1]
    return np.concatenate([v[(hq // (H // HKV)) * HD:(hq // (H // HKV) + 1) * HD]
                           for hq in range(H)])


@pytest.mark.parametrize("kv_f16", [False, True])
def test_one_position_attention_returns_v(orc, kv_f16):
    cfg = dict(CFG, n_layer=1)
    w = modelgen.host_model(orc, cfg, seed=22)
    w["blk.0.ffn_down"] = zero_like(orc, w, "blk.0.ffn_down")
    E, QD = cfg["n_embd"], cfg["n_head"] * cfg["head_dim"]
    tok = 123
    e = embed(orc, cfg, w, tok)
    att = _layer0_v_path(orc, cfg, w, e)
    if kv_f16:
        att = att.astype(np.float32).astype(np.float16).astype(np.float64)
    x1 = e + deq(orc, w, "blk.0.attn_output", QD, E) @ att
    got = orc.Model(cfg, w, kv_f16=kv_f16).forward([tok])
    assert rel(got, head(orc, cfg, w, x1)) < TOL
    # q and k cannot matter: the one softmax weight is exactly 1
    w2 = dict(w)
    for n in ("attn_q", "attn_k"):
        t, arr = w[n.join(["blk.0.", ""])]
        w2["blk.0." + n] = (t, orc.gen_weight(t, 999 + len(n), arr.size // (E // 256 * orc.TYPE_SIZE[t]), E, mode=1))
    w2["blk.0.bq"] = (F32, -w["blk.0.bq"][1])
    got2 = orc.Model(cfg, w2, kv_f16=kv_f16).forward([tok])
    assert np.array_equal(got.view(np.uint32), got2.view(np.uint32))


def test_identical_value_rows_make_attention_history_free(orc):
    """W_v = 0: every cached value row is bv, the softmax weights sum to 1, so
    the attention output is bv at every position; with ffn_down = 0 each
    position's logits depend on its own token only."""
    cfg = dict(CFG, n_layer=1)
    w = modelgen.host_model(orc, cfg, seed=23)
    w["blk.0.attn_v"] = zero_like(orc, w, "blk.0.attn_v")
    w["blk.0.ffn_down"] = zero_like(orc, w, "blk.0.ffn_down")
    E, H, HKV, HD = cfg["n_embd"], cfg["n_head"], cfg["n_head_kv"], cfg["head_dim"]
    bv = np.asarray(w["blk.0.bv"][1], np.float64)
    att = np.concatenate([bv[(hq // (H // HKV)) * HD:(hq // (H // HKV) + 1) * HD]
                          for hq in range(H)])
    o = deq(orc, w, "blk.0.attn_output", H * HD, E) @ att
    m = orc.Model(cfg, w, kv_f16=False)
    for tok in (5, 17, 300, 2, 99, 17):
        got = m.forward([tok])
        assert rel(got, head(orc, cfg, w, embed(orc, cfg, w, tok) + o)) < TOL


def test_ffn_only_layer_closed_form(orc):
    cfg = dict(CFG, n_layer=1)
    w = modelgen.host_model(orc, cfg, seed=24)
    w["blk.0.attn_output"] = zero_like(orc, w, "blk.0.attn_output")
    E, FF = cfg["n_embd"], cfg["n_ff"]
    m = orc.Model(cfg, w)
    for tok in (9, 250, 9):
        e = embed(orc, cfg, w, tok)
        h = rms(e, w["blk.0.ffn_norm"][1], cfg["rms_eps"])
        g = deq(orc, w, "blk.0.ffn_gate", E, FF) @ h
        u = deq(orc, w, "blk.0.ffn_up", E, FF) @ h
        x = e + deq(orc, w, "blk.0.ffn_down", FF, E) @ (silu(g) * u)
        assert rel(m.forward([tok]), head(orc, cfg, w, x)) < TOL


def test_q8_0_weights_take_the_int8_activation_path(orc):
    """all-Q8_0 weights with zero mixers: the head multiplies the Q8_0
    rounding (half to even) of rmsnorm(x) * output_norm, matmul_q8_0_actq
    (its integer block sums are pinned by brute force in test_oracle.py)"""
    w = modelgen.host_model(orc, CFG, seed=25, mix=modelgen.ALL_Q8_0)
    for l in range(CFG["n_layer"]):
        for n in ("attn_output", "ffn_down"):
            w[f"blk.{l}.{n}"] = zero_like(orc, w, f"blk.{l}.{n}")
    tok = 44
    x = embed(orc, CFG, w, tok).astype(np.float32)
    hn = orc.rmsnorm_scale(x, w["output_norm"][1], CFG["rms_eps"])
    t, arr = w["output"]
    want = orc.matvec_q8_0_actq(arr, CFG["n_embd"], CFG["vocab"], hn, half_even=True)
    got = orc.Model(CFG, w).forward([tok])
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    f32 = orc.Model(CFG, w, q8_actq=False).forward([tok])
    assert not np.array_equal(f32, got) and rel(f32, got) < 0.1


# --------------------------------------------------------------------------
# hybrid forward: one delta-net layer
# --------------------------------------------------------------------------
HY1 = dict(modelgen.HY_TINY, n_layer=1, full_attn_interval=2, ctx=16)


def _dn_inputs(orc, cfg, w, e):
    """h, conv input, z and the gates of layer 0 for a token with embedding e"""
    E, D, KH, VH = cfg["n_embd"], cfg["dn_state"], cfg["dn_k_heads"], cfg["dn_v_heads"]
    CD = modelgen.hy_conv_dim(cfg)
    h = rms(e, w["blk.0.attn_norm"][1], cfg["rms_eps"])
    cin = deq(orc, w, "blk.0.ssm_qkv", E, CD) @ h
    z = deq(orc, w, "blk.0.ssm_gate", E, VH * D) @ h
    al = np.asarray(w["blk.0.ssm_alpha"][1], np.float64).reshape(VH, E) @ h
    be = np.asarray(w["blk.0.ssm_beta"][1], np.float64).reshape(VH, E) @ h
    a = np.asarray(w["blk.0.ssm_a"][1], np.float64)
    dt = np.asarray(w["blk.0.ssm_dt"][1], np.float64)
    g = a * np.log1p(np.exp(al + dt))
    beta = 1.0 / (1.0 + np.exp(-be))
    return h, cin, z, g, beta


def _qkv_heads(cfg, conv_out):
    D, KH, VH = cfg["dn_state"], cfg["dn_k_heads"], cfg["dn_v_heads"]
    c = silu(conv_out)
    eps = cfg["rms_eps"]
    q = c[:KH * D].reshape(KH, D)
    k = c[KH * D:2 * KH * D].reshape(KH, D)
    v = c[2 * KH * D:].reshape(VH, D)
    q = q / np.sqrt((q * q).sum(1, keepdims=True) + eps)
    k = k / np.sqrt((k * k).sum(1, keepdims=True) + eps)
    return q, k, v


def _gated_out(orc, cfg, w, o, z):
    D, VH, E = cfg["dn_state"], cfg["dn_v_heads"], cfg["n_embd"]
    nw = np.asarray(w["blk.0.ssm_norm"][1], np.float64)
    y = np.concatenate([rms(o[hh], nw, cfg["rms_eps"]) * silu(z[hh * D:(hh + 1) * D])
                        for hh in range(VH)])
    return deq(orc, w, "blk.0.ssm_out", VH * D, E) @ y


@pytest.mark.parametrize("taps", ["random", "one-hot-previous"])
def test_delta_rule_two_steps_from_zero_state(orc, taps):
    cfg = HY1
    w = modelgen.hybrid_host_model(orc, cfg, seed=26)
    w["blk.0.ffn_down"] = zero_like(orc, w, "blk.0.ffn_down")
    D, KH, VH, W = cfg["dn_state"], cfg["dn_k_heads"], cfg["dn_v_heads"], cfg["dn_conv"]
    CD = modelgen.hy_conv_dim(cfg)
    if taps != "random":
        cw = np.zeros((CD, W), np.float32)
        cw[:, W - 2] = 1.0  # the conv output is the previous token's input
        w["blk.0.ssm_conv"] = (F32, cw.ravel())
    cw = np.asarray(w["blk.0.ssm_conv"][1], np.float64).reshape(CD, W)
    m = orc.HybridModel(cfg, w)
    t1, t2 = 31, 402
    e1, e2 = embed(orc, cfg, w, t1), embed(orc, cfg, w, t2)
    _, c1, z1, g1, b1 = _dn_inputs(orc, cfg, w, e1)
    _, c2, z2, g2, b2 = _dn_inputs(orc, cfg, w, e2)
    q1, k1, v1 = _qkv_heads(cfg, cw[:, W - 1] * c1)
    q2, k2, v2 = _qkv_heads(cfg, cw[:, W - 2] * c1 + cw[:, W - 1] * c2)
    sd = np.sqrt(D)
    o1 = np.stack([b1[h] * (k1[h % KH] @ q1[h % KH]) * v1[h] / sd for h in range(VH)])
    o2 = np.stack([(np.exp(g2[h]) * b1[h] * (k1[h % KH] @ q2[h % KH]) * v1[h]
                    + b2[h] * (k2[h % KH] @ q2[h % KH])
                    * (v2[h] - np.exp(g2[h]) * b1[h] * (k1[h % KH] @ k2[h % KH]) * v1[h])) / sd
                   for h in range(VH)])
    if taps == "random":
        want1 = head(orc, cfg, w, e1 + _gated_out(orc, cfg, w, o1, z1))
        assert rel(m.forward([t1]), want1) < 1e-4
    else:
        # q = k = v = 0 for the first token: the layer adds nothing
        assert rel(m.forward([t1]), head(orc, cfg, w, e1)) < TOL
    want2 = head(orc, cfg, w, e2 + _gated_out(orc, cfg, w, o2, z2))
    assert rel(m.forward([t2]), want2) < 1e-4


def test_hybrid_zero_mixers_give_embedding_then_head(orc):
    cfg = modelgen.HY_TINY
    w = modelgen.hybrid_host_model(orc, cfg, seed=27)
    for l in range(cfg["n_layer"]):
        names = ["ffn_down", "attn_output" if modelgen.hy_is_full(cfg, l) else "ssm_out"]
        for n in names:
            w[f"blk.{l}.{n}"] = zero_like(orc, w, f"blk.{l}.{n}")
    m = orc.HybridModel(cfg, w)
    for tok in (1, 300, 45, 1, 8):
        assert rel(m.forward([tok]), head(orc, cfg, w, embed(orc, cfg, w, tok))) < TOL
