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
  (weights.rs:113-117) bit for bit;
* the hybrid's gated attention: with one cached position the mixer is
  W_o (sigmoid(gate_h) * v_{h/rep}), the gate being rows [HD, 2HD) of head h's
  Q block, and the query half, attn_k, the norms and RoPE cannot move a bit;
  QK-norm makes each head's query and each KV head's key scale-free; q and k
  past rope_dim are not turned; a single adjacent pair gives the score
  (cos(d) q.k + sin(d) (q0 k1 - q1 k0)) / sqrt(HD), d = (t - j) f_i, at the
  closed-form frequencies f_0 = 1 and f_{rope_dim/4} = base^(-1/2).

Each reduction fails for a plausible mistake in the forward: residual
replaced instead of added, wrong norm weight, head on the wrong token, GQA
head mapping, unnormalised softmax, swapped gate / up, state transposed,
decay not applied or applied as g, sign of the delta correction, conv taps
reversed or shifted the wrong way, key head chosen by division instead of
modulo, and for the gated attention: query and gate halves swapped, the
query norm taken over 2 HD, no key norm or the query's norm weight on k, the
sign of the rotation, the frequency exponent over head_dim, q and k rotated
at different positions, the whole head rotated, the gate left out or taken
as tanh, the query-to-KV-head map by modulo (each fails a test here)."""
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


# --------------------------------------------------------------------------
# hybrid forward: the gated full-attention layers
# (resident_forward.rs:3865-3917; gate_quant.comp:39-46; dn_norm.comp:6-8;
# rope.comp:1-32; freq table gpu.rs:540-547)
# --------------------------------------------------------------------------
# every layer full attention, partial RoPE (32 of 64 dims), GQA 2:1
HYA = dict(modelgen.HY_TINY, n_layer=1, full_attn_interval=1, ctx=16)


def _q4k_rows(arr, n_in):
    return arr.reshape(-1, n_in // 256 * 144)


def _zero_rows(w, name, n_in, rows):
    t, arr = w[name]
    assert t == Q4_K
    a = arr.copy()
    _q4k_rows(a, n_in)[rows] = 0
    w[name] = (t, a)


def _double_rows(w, name, n_in, rows):
    """multiplies Q4_K rows by exactly 2: each super-block's f16 d and dmin
    (its first 4 bytes) get one more in the exponent"""
    t, arr = w[name]
    assert t == Q4_K
    a = arr.copy()
    r = _q4k_rows(a, n_in)
    for row in rows:
        sb = r[row].reshape(-1, 144)
        h = sb[:, :4].copy().view(np.uint16)
        e = (h >> 10) & 0x1F
        assert np.all((e > 0) & (e < 30) | (h == 0))
        h = np.where(h == 0, h, h + np.uint16(0x400)).astype(np.uint16)
        sb[:, :4] = h.view(np.uint8).reshape(-1, 4)
        r[row] = sb.ravel()
    w[name] = (t, a)


def _head_rows(cfg, hh, half):
    """rows of attn_q that hold head hh's query (half 0) or gate (half 1)"""
    HD = cfg["head_dim"]
    s = hh * 2 * HD + half * HD
    return np.arange(s, s + HD)


def _attn_inputs(orc, cfg, w, e, l=0):
    """h, the raw per-head query / gate rows, k and v of attention layer l"""
    E, H, HKV, HD = cfg["n_embd"], cfg["n_head"], cfg["n_head_kv"], cfg["head_dim"]
    h = rms(e, w[f"blk.{l}.attn_norm"][1], cfg["rms_eps"])
    qg = deq(orc, w, f"blk.{l}.attn_q", E, 2 * H * HD) @ h
    qg = qg.reshape(H, 2, HD)
    k = (deq(orc, w, f"blk.{l}.attn_k", E, HKV * HD) @ h).reshape(HKV, HD)
    v = (deq(orc, w, f"blk.{l}.attn_v", E, HKV * HD) @ h).reshape(HKV, HD)
    return h, qg[:, 0], qg[:, 1], k, v


def _rotate(x, pos, cfg):
    """adjacent pairs (2i, 2i+1), i < rope_dim/2, turned by pos * base^(-2i/rope_dim);
    the dims from rope_dim on are left alone"""
    x = np.array(x, np.float64)
    for i in range(cfg["rope_dim"] // 2):
        th = pos * cfg["freq_base"] ** (-2.0 * i / cfg["rope_dim"])
        c, s = np.cos(th), np.sin(th)
        a, b = x[2 * i], x[2 * i + 1]
        x[2 * i], x[2 * i + 1] = a * c - b * s, a * s + b * c
    return x


def _attn_layer_closed_form(orc, cfg, w, embs, l=0):
    """float64 output of attention layer l (before attn_output) for the last of
    the tokens whose embeddings (inputs of the layer) are embs, every one cached"""
    H, HKV, HD = cfg["n_head"], cfg["n_head_kv"], cfg["head_dim"]
    rep, eps = H // HKV, cfg["rms_eps"]
    qn = np.asarray(w[f"blk.{l}.q_norm"][1], np.float64)
    kn = np.asarray(w[f"blk.{l}.k_norm"][1], np.float64)
    ks, vs = [], []
    for pos, e in enumerate(embs):
        _, q, gate, k, v = _attn_inputs(orc, cfg, w, e, l)
        ks.append([_rotate(rms(k[g], kn, eps), pos, cfg) for g in range(HKV)])
        vs.append(v)
    t = len(embs) - 1
    out = []
    for hh in range(H):
        g = hh // rep
        qr = _rotate(rms(q[hh], qn, eps), t, cfg)
        s = np.array([qr @ ks[j][g] for j in range(t + 1)]) / np.sqrt(HD)
        p = np.exp(s - s.max())
        p /= p.sum()
        att = sum(p[j] * vs[j][g] for j in range(t + 1))
        out.append(att / (1.0 + np.exp(-gate[hh])))
    return np.concatenate(out)


@pytest.mark.parametrize("kv_f16", [False, True])
def test_gated_attention_one_position_is_gated_v(orc, kv_f16):
    """one cached position: the softmax weight is exactly 1, so the mixer is
    W_o (sigmoid(gate_h) * v_{h/rep}), the gate being rows [HD, 2HD) of head h's
    Q block; the query half, attn_k, the q / k norms and RoPE cannot move a bit"""
    cfg = HYA
    w = modelgen.hybrid_host_model(orc, cfg, seed=31)
    w["blk.0.ffn_down"] = zero_like(orc, w, "blk.0.ffn_down")
    E, H, HKV, HD = cfg["n_embd"], cfg["n_head"], cfg["n_head_kv"], cfg["head_dim"]
    tok = 77
    e = embed(orc, cfg, w, tok)
    _, _, gate, _, v = _attn_inputs(orc, cfg, w, e)
    if kv_f16:
        v = v.astype(np.float32).astype(np.float16).astype(np.float64)
    att = np.concatenate([v[hh // (H // HKV)] / (1.0 + np.exp(-gate[hh])) for hh in range(H)])
    x1 = e + deq(orc, w, "blk.0.attn_output", H * HD, E) @ att
    got = orc.HybridModel(cfg, w, kv_f16=kv_f16).forward([tok])
    assert rel(got, head(orc, cfg, w, x1)) < TOL

    w2 = dict(w)
    t, arr = w["blk.0.attn_q"]
    other = orc.gen_weight(t, 4242, 2 * H * HD, E, mode=1)
    a = arr.copy()
    qrows = np.concatenate([_head_rows(cfg, hh, 0) for hh in range(H)])
    _q4k_rows(a, E)[qrows] = _q4k_rows(other, E)[qrows]
    w2["blk.0.attn_q"] = (t, a)
    tk, ak = w["blk.0.attn_k"]
    w2["blk.0.attn_k"] = (tk, orc.gen_weight(tk, 4343, HKV * HD, E, mode=1))
    w2["blk.0.q_norm"] = (F32, orc.gen_uniform(4444, HD, -2.0, 2.0))
    w2["blk.0.k_norm"] = (F32, orc.gen_uniform(4545, HD, -2.0, 2.0))
    got2 = orc.HybridModel(dict(cfg, freq_base=3.0), w2, kv_f16=kv_f16).forward([tok])
    assert np.array_equal(got.view(np.uint32), got2.view(np.uint32))
    # while the gate half does matter
    w3 = dict(w)
    _double_rows(w3, "blk.0.attn_q", E, _head_rows(cfg, 1, 1))
    assert rel(orc.HybridModel(cfg, w3, kv_f16=kv_f16).forward([tok]), got) > 1e-3


def test_qk_norm_makes_each_head_scale_free(orc):
    """QK-norm normalises each head's HD query dims on their own (dn_norm mode 2,
    stride 2 HD): doubling one head's query rows, or one KV head's key rows,
    leaves the logits unchanged up to the eps term; doubling a gate half moves them"""
    cfg = HYA
    E, HD = cfg["n_embd"], cfg["head_dim"]
    w = modelgen.hybrid_host_model(orc, cfg, seed=32)
    toks = [5, 300, 17, 260]

    def run(ww):
        return orc.HybridModel(cfg, ww, kv_f16=False).forward(toks)

    base = run(w)
    wq = dict(w)
    _double_rows(wq, "blk.0.attn_q", E, _head_rows(cfg, 1, 0))
    assert rel(run(wq), base) < 1e-6
    wk = dict(w)
    _double_rows(wk, "blk.0.attn_k", E, np.arange(HD, 2 * HD))
    assert rel(run(wk), base) < 1e-6
    wg = dict(w)
    _double_rows(wg, "blk.0.attn_q", E, _head_rows(cfg, 1, 1))
    assert rel(run(wg), base) > 1e-3
    # and the scores do matter here (so the invariance above is not vacuous)
    wz = dict(w)
    _zero_rows(wz, "blk.0.attn_q", E, _head_rows(cfg, 1, 0))
    assert rel(run(wz), base) > 1e-3


def test_partial_rope_leaves_dims_past_rope_dim_alone(orc):
    """q and k non-zero only in dims >= rope_dim: RoPE turns nothing, the scores
    do not depend on position, and the layer is the plain QK-normed softmax
    attention (closed form over 5 cached positions)"""
    cfg = HYA
    E, H, HKV, HD, RD = (cfg[k] for k in ("n_embd", "n_head", "n_head_kv", "head_dim", "rope_dim"))
    w = modelgen.hybrid_host_model(orc, cfg, seed=33)
    w["blk.0.ffn_down"] = zero_like(orc, w, "blk.0.ffn_down")
    _zero_rows(w, "blk.0.attn_q", E, np.concatenate([hh * 2 * HD + np.arange(RD) for hh in range(H)]))
    _zero_rows(w, "blk.0.attn_k", E, np.concatenate([g * HD + np.arange(RD) for g in range(HKV)]))
    toks = [9, 410, 33, 9, 128]
    embs = [embed(orc, cfg, w, t) for t in toks]
    m = orc.HybridModel(cfg, w, kv_f16=False)
    WO = deq(orc, w, "blk.0.attn_output", H * HD, E)
    for n in range(1, len(toks) + 1):
        got = m.forward([toks[n - 1]])
        att = _attn_layer_closed_form(orc, cfg, w, embs[:n])
        assert rel(got, head(orc, cfg, w, embs[n - 1] + WO @ att)) < 1e-5
    # no rotation at all: the same closed form with the angles set to zero
    assert np.allclose(_rotate(np.arange(HD, dtype=np.float64) * (np.arange(HD) >= RD), 7, cfg),
                       np.arange(HD) * (np.arange(HD) >= RD))


@pytest.mark.parametrize("pair", [0, 8])
def test_rope_pair_scores_expanded_by_hand(orc, pair):
    """q and k non-zero only in the adjacent pair (2i, 2i+1): the score of query
    position t against key position j is
    (cos(d) (q.k) + sin(d) (q0 k1 - q1 k0)) / sqrt(HD), d = (t - j) * f_i,
    with f_0 = 1 and f_{rope_dim/4} = base^(-1/2) = 1/4 at base 16 (the
    1/base^(2i/rope_dim) table at closed-form points)"""
    cfg = dict(HYA, freq_base=16.0)
    E, H, HKV, HD, RD = (cfg[k] for k in ("n_embd", "n_head", "n_head_kv", "head_dim", "rope_dim"))
    assert pair in (0, RD // 4)
    f = 1.0 if pair == 0 else 0.25
    w = modelgen.hybrid_host_model(orc, cfg, seed=34)
    w["blk.0.ffn_down"] = zero_like(orc, w, "blk.0.ffn_down")
    keep = (np.arange(HD) // 2) == pair
    _zero_rows(w, "blk.0.attn_q", E, np.concatenate([hh * 2 * HD + np.nonzero(~keep)[0]
                                                     for hh in range(H)]))
    _zero_rows(w, "blk.0.attn_k", E, np.concatenate([g * HD + np.nonzero(~keep)[0]
                                                     for g in range(HKV)]))
    toks = [21, 300, 4, 77, 200, 21]
    embs = [embed(orc, cfg, w, t) for t in toks]
    qn = np.asarray(w["blk.0.q_norm"][1], np.float64)
    kn = np.asarray(w["blk.0.k_norm"][1], np.float64)
    eps, rep = cfg["rms_eps"], H // HKV
    m = orc.HybridModel(cfg, w, kv_f16=False)
    WO = deq(orc, w, "blk.0.attn_output", H * HD, E)
    ins = [_attn_inputs(orc, cfg, w, e) for e in embs]
    i0, i1 = 2 * pair, 2 * pair + 1
    moved = 0.0
    for t in range(len(toks)):
        got = m.forward([toks[t]])
        out = []
        for hh in range(H):
            g = hh // rep
            q = rms(ins[t][1][hh], qn, eps)
            s = []
            for j in range(t + 1):
                k = rms(ins[j][3][g], kn, eps)
                d = (t - j) * f
                dot, cross = q[i0] * k[i0] + q[i1] * k[i1], q[i0] * k[i1] - q[i1] * k[i0]
                s.append((np.cos(d) * dot + np.sin(d) * cross) / np.sqrt(HD))
                moved = max(moved, abs(np.sin(d) * cross) / np.sqrt(HD))
            s = np.array(s)
            p = np.exp(s - s.max())
            p /= p.sum()
            att = sum(p[j] * ins[j][4][g] for j in range(t + 1))
            out.append(att / (1.0 + np.exp(-ins[t][2][hh])))
        want = head(orc, cfg, w, embs[t] + WO @ np.concatenate(out))
        assert rel(got, want) < 1e-5, t
    assert moved > 0.1  # the rotation term is not negligible in these scores


def test_mixed_layers_delta_net_then_attention(orc):
    """layer 0 gated delta net, layer 1 gated attention (full_attn_interval 2):
    for the first token, x1 = e + the delta rule from a zero state
    (beta (k.q) v / sqrt(d), gated), then one cached position in layer 1
    (gated v), each layer's FFN zeroed"""
    cfg = dict(modelgen.HY_TINY, n_layer=2, full_attn_interval=2, ctx=16)
    w = modelgen.hybrid_host_model(orc, cfg, seed=35)
    for l in range(2):
        w[f"blk.{l}.ffn_down"] = zero_like(orc, w, f"blk.{l}.ffn_down")
    D, KH, VH, W = cfg["dn_state"], cfg["dn_k_heads"], cfg["dn_v_heads"], cfg["dn_conv"]
    E, H, HKV, HD = cfg["n_embd"], cfg["n_head"], cfg["n_head_kv"], cfg["head_dim"]
    CD = modelgen.hy_conv_dim(cfg)
    tok = 140
    e = embed(orc, cfg, w, tok)
    _, c1, z1, _, b1 = _dn_inputs(orc, cfg, w, e)
    cw = np.asarray(w["blk.0.ssm_conv"][1], np.float64).reshape(CD, W)
    q1, k1, v1 = _qkv_heads(cfg, cw[:, W - 1] * c1)
    o1 = np.stack([b1[h] * (k1[h % KH] @ q1[h % KH]) * v1[h] / np.sqrt(D) for h in range(VH)])
    x1 = e + _gated_out(orc, cfg, w, o1, z1)
    _, _, gate, _, v = _attn_inputs(orc, cfg, w, x1, l=1)
    v = v.astype(np.float32).astype(np.float16).astype(np.float64)
    att = np.concatenate([v[hh // (H // HKV)] / (1.0 + np.exp(-gate[hh])) for hh in range(H)])
    x2 = x1 + deq(orc, w, "blk.1.attn_output", H * HD, E) @ att
    got = orc.HybridModel(cfg, w).forward([tok])
    assert rel(got, head(orc, cfg, w, x2)) < 1e-4
