"""Pins the CPU oracle before it is trusted as the parity checker.

Known answers come from the reference's own unit tests (cited per test); the
Q5_K block is the llama.cpp gguf-py golden fixture the reference commits; the
rest is checked against independent restatements (numpy float16, the numpy
element-wise dequant in npref.py, float64 dots) or closed forms.
"""
import json
import math
import os

import numpy as np
import pytest

import npref

HERE = os.path.dirname(os.path.abspath(__file__))
F32, F16, Q4_0, Q8_0, Q4_K, Q5_K, Q6_K = 0, 1, 2, 8, 12, 13, 14


def f16b(v: float) -> list:
    h = int(np.array([v], dtype=np.float16).view(np.uint16)[0])
    return [h & 0xFF, h >> 8]


# --------------------------------------------------------------------------
# f16 <-> f32
# --------------------------------------------------------------------------
def test_f16_to_f32_exhaustive(orc):
    codes = np.arange(65536, dtype=np.uint32)
    ours = np.array([orc.f16_to_f32(int(c)) for c in codes], dtype=np.float32)
    ref = codes.astype(np.uint16).view(np.float16).astype(np.float32)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(ours), nan)
    assert np.array_equal(ours[~nan].view(np.uint32), ref[~nan].view(np.uint32))


def test_f32_to_f16_round_to_nearest_even(orc):
    rng = np.random.default_rng(7)
    vals = np.concatenate([
        rng.standard_normal(4000).astype(np.float32) * 10.0 ** rng.integers(-9, 6, 4000),
        np.array([0.0, -0.0, 65504.0, 65519.99, 65520.0, 1e9, -1e9, 5.96e-8, 2.98e-8,
                  2.99e-8, 1e-10, 6.1e-5, 6.097e-5, 1.0 + 2 ** -11, 1.0 + 3 * 2 ** -11,
                  np.inf, -np.inf], dtype=np.float32)])
    ours = np.array([orc.f32_to_f16(float(v)) for v in vals], dtype=np.uint16)
    ref = vals.astype(np.float16).view(np.uint16)
    assert np.array_equal(ours, ref)


# --------------------------------------------------------------------------
# dequant known answers (crates/ggml-cpu/src/dequant.rs:269-469)
# --------------------------------------------------------------------------
def test_q8_0_single_block(orc):  # dequant.rs:297-309
    qs = [1, 0xFF] + [0] * 30
    out = orc.dequant(Q8_0, bytes(f16b(1.0) + qs))
    assert out.size == 32 and out[0] == 1.0 and out[1] == -1.0 and np.all(out[2:] == 0)


def test_q8_0_scale_applied(orc):  # dequant.rs:311-319
    out = orc.dequant(Q8_0, bytes(f16b(2.0) + [3] + [0] * 31))
    assert out[0] == 6.0


def test_q4_0_single_block(orc):  # dequant.rs:332-351
    qs = [0x89] + [0x88] * 15
    out = orc.dequant(Q4_0, bytes(f16b(1.0) + qs))
    assert out[0] == 1.0 and np.all(out[1:] == 0)


def test_q4_k_two_active_sub_blocks(orc):  # dequant.rs:366-394
    scales = [8, 4] + [0] * 10
    out = orc.dequant(Q4_K, bytes(f16b(1.0) + f16b(1.0) + scales + [0x22] * 128))
    exp = np.zeros(256, np.float32)
    exp[:32], exp[32:64] = 16.0, 8.0
    assert np.array_equal(out, exp)


def test_q6_k_all_zero_ql_qh(orc):  # dequant.rs:410-464
    scales = [1, 0] * 8
    out = orc.dequant(Q6_K, bytes([0] * 128 + [0] * 64 + scales + f16b(1.0)))
    for base in (0, 128):
        for l in range(32):
            for off in (0, 32, 64, 96):
                assert out[base + l + off] == (-32.0 if l < 16 else 0.0)


def test_q6_k_one_hot_quant_bits(orc):
    """Every single set bit of ql (128 bytes) and qh (64 bytes) with d = 1 and
    all scales 1: exactly one element moves from -32 to 2^k - 32.  Positions
    from the GGUF Q6_K layout: per 128-element half n, ql[64n + j] low nibble
    is quant bits 0-3 of element 128n + j and its high nibble of element
    128n + j + 64; qh[32n + l] bit pair p is quant bits 4-5 of element
    128n + l + 32p."""
    base = [0] * 128 + [0] * 64 + [1] * 16 + f16b(1.0)
    for byte in range(192):
        for bit in range(8):
            blk = list(base)
            blk[byte] = 1 << bit
            out = orc.dequant(Q6_K, bytes(blk))
            if byte < 128:
                n, j = byte // 64, byte % 64
                elem = 128 * n + j + (64 if bit >= 4 else 0)
                k = bit % 4
            else:
                n, l = (byte - 128) // 32, (byte - 128) % 32
                elem = 128 * n + l + 32 * (bit // 2)
                k = 4 + bit % 2
            exp = np.full(256, -32.0, np.float32)
            exp[elem] = float((1 << k) - 32)
            assert np.array_equal(out, exp), (byte, bit)


def test_q6_k_one_hot_scale_slots(orc):
    """One nonzero int8 scale s (slot i) with d = 1 and all quants 0: exactly
    the 16 elements of that slot read -32 * s; slot 8n + 2p + m covers
    elements 128n + 32p + 16m .. +15."""
    for slot in range(16):
        for s in (1, -1, 127, -128):
            sc = [0] * 16
            sc[slot] = s & 0xFF
            out = orc.dequant(Q6_K, bytes([0] * 192 + sc + f16b(1.0)))
            n, r = slot // 8, slot % 8
            e0 = 128 * n + 32 * (r // 2) + 16 * (r % 2)
            exp = np.zeros(256, np.float32)
            exp[e0:e0 + 16] = -32.0 * s
            assert np.array_equal(out, exp), (slot, s)


@pytest.mark.parametrize("t,bad", [(Q8_0, 33), (Q4_0, 17), (Q4_K, 143), (Q5_K, 175),
                                   (Q6_K, 209)])
def test_bad_size_is_an_error(orc, t, bad):  # dequant.rs BadSize arms
    with pytest.raises(ValueError):
        orc.dequant(t, bytes(bad))


def test_q5_k_gguf_py_golden_block(orc):  # dequant.rs:472-548
    fx = json.load(open(os.path.join(HERE, "golden", "q5_k_gguf_py_block.json")))
    out = orc.dequant(Q5_K, bytes(fx["raw"]))
    assert out.size == 256
    for i, v in fx["spots"]:
        assert abs(out[i] - v) < fx["spot_tol"], (i, out[i], v)
    assert abs(out.astype(np.float64).sum() - fx["sum"]) < fx["sum_tol"]
    # the numpy restatement agrees bit for bit on the real block too
    assert np.array_equal(out.view(np.uint32), npref.dequant(Q5_K, np.array(fx["raw"], np.uint8)).view(np.uint32))


# --------------------------------------------------------------------------
# dequant vs the independent numpy restatement (bit exact), random blocks
# --------------------------------------------------------------------------
@pytest.mark.parametrize("t", [Q8_0, Q4_0, Q4_K, Q5_K, Q6_K, F16, F32])
def test_dequant_matches_numpy_restatement(orc, t):
    rng = np.random.default_rng(100 + t)
    ts = orc.TYPE_SIZE[t]
    raw = rng.integers(0, 256, size=ts * 512, dtype=np.uint8)
    if t in (Q8_0, Q4_0):
        for b in range(512):  # sane f16 scales (random bytes may be NaN/inf)
            raw[b * ts:b * ts + 2] = f16b(float(rng.uniform(-2, 2)))
    elif t in (Q4_K, Q5_K):
        for b in range(512):
            raw[b * ts:b * ts + 2] = f16b(float(rng.uniform(1e-3, 1e-1)))
            raw[b * ts + 2:b * ts + 4] = f16b(float(rng.uniform(1e-3, 1e-1)))
    elif t == Q6_K:
        for b in range(512):
            raw[b * ts + 208:b * ts + 210] = f16b(float(rng.uniform(-1e-1, 1e-1)))
    elif t == F32:
        raw = rng.standard_normal(512).astype(np.float32).view(np.uint8)
    elif t == F16:
        raw = rng.standard_normal(512).astype(np.float16).view(np.uint8)
    ours = orc.dequant(t, raw)
    ref = npref.dequant(t, raw)
    assert np.array_equal(ours.view(np.uint32), ref.view(np.uint32))


def test_q4_k_scale_unpack_brute_force(orc):
    """Every 6-bit (sc, m) value in every one of the 8 sub-block slots, via a
    one-hot nibble pattern: out[sub-block s] = d*sc[s]*1 - dmin*m[s]."""
    rng = np.random.default_rng(3)
    for trial in range(64):
        sc = rng.integers(0, 64, 8)
        m = rng.integers(0, 64, 8)
        sc[trial % 8] = trial  # walk every value through every slot
        s = np.zeros(12, np.int64)
        s[0:4] = (sc[0:4] & 63) | ((sc[4:8] >> 4) << 6)
        s[4:8] = (m[0:4] & 63) | ((m[4:8] >> 4) << 6)
        s[8:12] = (sc[4:8] & 15) | ((m[4:8] & 15) << 4)
        blk = bytes(f16b(1.0) + f16b(1.0) + [int(v) for v in s] + [0x11] * 128)
        out = orc.dequant(Q4_K, blk)
        for sub in range(8):
            assert np.all(out[32 * sub:32 * sub + 32] == float(sc[sub]) - float(m[sub]))


# --------------------------------------------------------------------------
# matvec (dequant + ops::matmul, ops.rs:78-101)
# --------------------------------------------------------------------------
def test_matmul_known_answers(orc):  # ops.rs:1098-1121 (F32 weights)
    w = np.array([1, 0, 0, 1], np.float32).view(np.uint8)
    assert list(orc.matvec(F32, w, 2, 2, np.array([5, 7], np.float32))) == [5.0, 7.0]
    w = np.array([2, 3], np.float32).view(np.uint8)
    assert list(orc.matvec(F32, w, 2, 1, np.array([5, 7], np.float32))) == [31.0]
    w = np.array([1, 1, 1, -1], np.float32).view(np.uint8)
    y = orc.matvec(F32, w, 2, 2, np.array([[1, 2], [3, 4]], np.float32))
    assert y.tolist() == [[3.0, -1.0], [7.0, -1.0]]


@pytest.mark.parametrize("t,n_in", [(Q8_0, 4864), (Q4_K, 5120), (Q5_K, 4096), (Q6_K, 512)])
def test_matvec_vs_f64_and_one_hot(orc, t, n_in):
    n_out = 16
    w = orc.gen_weight(t, 11, n_out, n_in)
    x = orc.gen_normal(5, n_in)
    y = orc.matvec(t, w, n_in, n_out, x)
    deq = orc.dequant(t, w).reshape(n_out, n_in).astype(np.float64)
    y64 = deq @ x.astype(np.float64)
    rel = np.linalg.norm(y - y64) / np.linalg.norm(y64)
    assert rel < 1e-5, rel
    # one-hot x selects a dequantized column exactly
    for col in (0, n_in // 2 + 3, n_in - 1):
        e = np.zeros(n_in, np.float32)
        e[col] = 1.0
        assert np.array_equal(orc.matvec(t, w, n_in, n_out, e), deq[:, col].astype(np.float32))
    # columns of a batched call equal single-column calls exactly
    xs = np.stack([orc.gen_normal(50 + c, n_in) for c in range(3)])
    yb = orc.matvec(t, w, n_in, n_out, xs)
    for c in range(3):
        assert np.array_equal(yb[c], orc.matvec(t, w, n_in, n_out, xs[c]))


def test_matvec_threads_do_not_change_bits(orc):
    w = orc.gen_weight(Q4_K, 1, 1000, 512)
    x = orc.gen_normal(2, 512)
    assert np.array_equal(orc.matvec(Q4_K, w, 512, 1000, x, threads=1),
                          orc.matvec(Q4_K, w, 512, 1000, x, threads=4))


def test_matvec_rejects_bad_shapes(orc):
    w = orc.gen_weight(Q4_K, 1, 4, 512)
    with pytest.raises(ValueError):
        orc.matvec(Q4_K, w, 500, 4, np.zeros(500, np.float32))
    with pytest.raises(ValueError):
        orc.matvec(Q4_K, w[:-1], 512, 4, np.zeros(512, np.float32))


# --------------------------------------------------------------------------
# generator
# --------------------------------------------------------------------------
def test_generator_distributions(orc):
    n = 4096
    q8 = orc.gen_blocks(Q8_0, 9, n).reshape(n, 34)
    d = q8[:, :2].copy().view(np.float16).astype(np.float32).ravel()
    assert d.min() >= 1e-3 * (1 - 1e-3) and d.max() <= 1e-2 * (1 + 1e-3)
    qs = q8[:, 2:].view(np.int8)
    assert qs.min() == -127 and qs.max() == 127
    q6 = orc.gen_blocks(Q6_K, 9, n).reshape(n, 210)
    sc = q6[:, 192:208].view(np.int8)
    assert sc.min() == -64 and sc.max() == 63
    # same (seed, block) -> same bytes regardless of the batch it is made in
    a = orc.gen_blocks(Q4_K, 77, 10, block0=0)
    b = orc.gen_blocks(Q4_K, 77, 3, block0=7)
    assert np.array_equal(a[7 * 144:], b)
    # centred mode: mins equal scales, dmin = f16(7.5 d): near zero-mean weights
    c = orc.gen_weight(Q4_K, 5, 64, 2048, mode=1)
    w = orc.dequant(Q4_K, c)
    assert abs(w.mean()) < 0.05 * w.std()
    blk = c.reshape(-1, 144)
    sc6, m6 = npref.kquant_scales(blk[:, 4:16])
    assert np.array_equal(sc6, m6)


def test_gen_normal_moments(orc):
    x = orc.gen_normal(1, 200000)
    assert abs(x.mean()) < 0.01 and abs(x.std() - 1) < 0.01


# --------------------------------------------------------------------------
# ops known answers (ops.rs:1065-1164)
# --------------------------------------------------------------------------
def test_rmsnorm_known_answer(orc):  # ops.rs:1065-1072
    out = orc.rmsnorm_scale(np.array([3.0, 4.0]), np.array([1.0, 1.0]), 0.0)
    s = 1.0 / math.sqrt(12.5)
    assert abs(out[0] - 3 * s) < 1e-6 and abs(out[1] - 4 * s) < 1e-6
    x = np.array([1, 2, 3, 4, 5, 6], np.float32)
    w = np.array([0.5, 2.0], np.float32)
    got = orc.rmsnorm_scale(x, w, 1e-5).reshape(3, 2)
    xr = x.reshape(3, 2).astype(np.float64)
    exp = xr / np.sqrt((xr * xr).mean(1, keepdims=True) + 1e-5) * w
    assert np.abs(got - exp).max() < 1e-6


def test_freq_table_and_rope_known_answers(orc):  # ops.rs:1123-1149
    fr = orc.freq_table(10000.0, 4)
    assert fr[0] == 1.0 and abs(fr[1] - 0.01) < 1e-9
    x = orc.rope_norm(np.array([1, 2, 3, 4], np.float32), 1, 1, 4, 4, fr, 0)
    assert np.abs(x - [1, 2, 3, 4]).max() < 1e-6
    x = orc.rope_norm(np.array([1, 0, 0, 0], np.float32), 1, 1, 4, 4, fr, 1)
    assert abs(x[0] - math.cos(1)) < 1e-6 and abs(x[1] - math.sin(1)) < 1e-6


def test_rope_is_a_rotation_of_adjacent_pairs(orc):
    rng = np.random.default_rng(0)
    x = rng.standard_normal(3 * 2 * 8).astype(np.float32)
    fr = orc.freq_table(1e6, 8)
    y = orc.rope_norm(x, 3, 2, 8, 8, fr, 17)
    xp, yp = x.reshape(-1, 2), y.reshape(-1, 2)
    assert np.allclose(np.hypot(xp[:, 0], xp[:, 1]), np.hypot(yp[:, 0], yp[:, 1]), rtol=1e-5)
    # pair i of token t rotates by (17+t)*freq[i]
    ang = np.arctan2(yp[:, 1], yp[:, 0]) - np.arctan2(xp[:, 1], xp[:, 0])
    t = np.repeat(np.arange(3), 2 * 4)
    i = np.tile(np.arange(4), 3 * 2)
    exp = (17 + t) * fr[i].astype(np.float64)
    assert np.allclose(np.angle(np.exp(1j * (ang - exp))), 0, atol=1e-4)


def test_swiglu_softmax_argmax(orc):  # ops.rs:1151-1164
    out = orc.swiglu(np.array([0.0, 2.0]), np.array([1.0, 3.0]))
    assert abs(out[0]) < 1e-6 and abs(out[1] - 3 * 2 / (1 + math.exp(-2))) < 1e-5
    z = orc.softmax(np.array([1.0, 2.0, 3.0]))
    assert abs(z.sum() - 1) < 1e-6 and z[2] > z[1] > z[0]
    assert orc.argmax(np.array([0.1, 0.9, 0.9, 0.2])) == 1


# --------------------------------------------------------------------------
# attention (attention.rs:174-260)
# --------------------------------------------------------------------------
def test_attention_known_answers(orc):
    out = orc.attention([1.0, 0.0], [0.5, 0.5], [9.0, 7.0], 1, 0, 1, 1, 2)
    assert abs(out[0] - 9) < 1e-6 and abs(out[1] - 7) < 1e-6
    out = orc.attention([1.0, 2.0], [3.0], [5.0], 1, 0, 2, 1, 1)
    assert abs(out[0] - 5) < 1e-6 and abs(out[1] - 5) < 1e-6
    out = orc.attention([1.0, 1.0], [0.0, 100.0], [2.0, 8.0], 2, 0, 1, 1, 1)
    assert abs(out[0] - 2) < 1e-6


def test_attention_matches_float64(orc):
    rng = np.random.default_rng(1)
    H, HKV, HD, n_tok, pos0 = 8, 2, 16, 3, 5
    T = pos0 + n_tok
    q = rng.standard_normal(n_tok * H * HD).astype(np.float32)
    k = rng.standard_normal(T * HKV * HD).astype(np.float32)
    v = rng.standard_normal(T * HKV * HD).astype(np.float32)
    out = orc.attention(q, k, v, n_tok, pos0, H, HKV, HD).reshape(n_tok, H, HD)
    K, V = k.reshape(T, HKV, HD).astype(np.float64), v.reshape(T, HKV, HD).astype(np.float64)
    Q = q.reshape(n_tok, H, HD).astype(np.float64)
    for t in range(n_tok):
        for h in range(H):
            s = K[:pos0 + t + 1, h // (H // HKV)] @ Q[t, h] / math.sqrt(HD)
            p = np.exp(s - s.max())
            p /= p.sum()
            assert np.abs(out[t, h] - p @ V[:pos0 + t + 1, h // (H // HKV)]).max() < 1e-5


# --------------------------------------------------------------------------
# delta-net primitives (delta_net.rs:133-255)
# --------------------------------------------------------------------------
def test_delta_net_known_answers(orc):
    assert abs(orc.lib().lrso_softplus(0.0) - math.log(2)) < 1e-6
    assert abs(orc.lib().lrso_softplus(50.0) - 50) < 1e-6
    sp = orc.lib().lrso_softplus(-30.0)
    assert 0 < sp < 1e-12
    x = orc.l2_norm_rows([3, 4, 0, 0, 5, 12, 0, 0], 4, 0.0).reshape(2, 4)
    assert np.allclose(np.linalg.norm(x, axis=1), 1, atol=1e-6) and abs(x[0, 0] - 0.6) < 1e-6
    # conv with state == direct causal convolution
    ch, dc, n = 3, 4, 6
    w = (np.arange(ch * dc) * 0.1 - 0.5).astype(np.float32)
    seq = [((np.arange(ch) + t * ch) * 0.25 - 1.0).astype(np.float32) for t in range(n)]
    st = np.zeros(ch * (dc - 1), np.float32)
    for t in range(n):
        out, st = orc.conv1d_step(st, seq[t], w, dc)
        for c in range(ch):
            exp = sum(seq[t + i - (dc - 1)][c] * w[c * dc + i]
                      for i in range(dc) if t + i - (dc - 1) >= 0)
            assert abs(out[c] - exp) < 1e-5
    # write (k,v) with unit k, read with q=k -> v/sqrt(d)
    d = 4
    k1 = np.array([1, 0, 0, 0], np.float32)
    v1 = np.array([0.5, -1.5, 2.0, 0.25], np.float32)
    out, st = orc.delta_net_step(np.zeros(d * d), k1, k1, v1, 0.0, 1.0)
    assert np.abs(out * 2 - v1).max() < 1e-6
    v1 = np.array([1, 2, 3, 4], np.float32)
    k2 = np.array([0, 1, 0, 0], np.float32)
    v2 = np.array([-1, 0, 1, 0], np.float32)
    _, st = orc.delta_net_step(np.zeros(d * d), k1, k1, v1, 0.0, 1.0)
    out, st = orc.delta_net_step(st, k2, k2, v2, math.log(0.5), 1.0)
    assert np.abs(out * 2 - v2).max() < 1e-6
    out, st = orc.delta_net_step(st, k1, k1, np.zeros(d), 0.0, 0.0)
    assert np.abs(out * 2 - v1 * 0.5).max() < 1e-5


# --------------------------------------------------------------------------
# dense forward (model.rs:99-266) vs a float64 numpy restatement
# --------------------------------------------------------------------------
@pytest.mark.parametrize("kv_f16", [False, True])
def test_forward_matches_float64_restatement(orc, kv_f16):
    import modelgen

    cfg = dict(modelgen.TINY, n_layer=2, ctx=16)
    w = modelgen.host_model(orc, cfg, seed=3)
    toks = [5, 17, 300, 2, 99]
    m = orc.Model(cfg, w, kv_f16=kv_f16)
    got = m.forward(toks)
    ref = npref.rms_forward64(cfg, w, toks, kv_f16=kv_f16)[-1]
    rel = np.linalg.norm(got - ref) / np.linalg.norm(ref)
    assert rel < 1e-4, rel
    assert len(m) == 5
    # one token at a time gives the same logits bit for bit (same per-row folds)
    m2 = orc.Model(cfg, w, kv_f16=kv_f16)
    for t in toks:
        last = m2.forward([t])
    assert np.array_equal(last, got)


def test_forward_context_overflow_and_bad_token(orc):
    import modelgen

    cfg = dict(modelgen.TINY, n_layer=1, ctx=4)
    m = orc.Model(cfg, modelgen.host_model(orc, cfg, seed=4))
    m.forward([1, 2, 3])
    with pytest.raises(ValueError):
        m.forward([4, 5])  # 3 + 2 > ctx: attention.rs:36-40
    with pytest.raises(ValueError):
        m.forward([cfg["vocab"]])


# --------------------------------------------------------------------------
# int8-activation Q8_0 path (ops.rs:284-385, 704-724, 728-886)
# --------------------------------------------------------------------------
def _q8_block(d_bits, qs):
    return np.array([d_bits & 0xFF, d_bits >> 8] + [q & 0xFF for q in qs], np.uint8)


def test_q8_quantize_ties_follow_each_rounding(orc):
    """max|x| = 127 makes d = 1 and 1/d = 1 exactly, so q = round(x): the
    AVX2 path (cvtps2dq) rounds ties to even, the scalar path away from 0."""
    x = np.zeros(32, np.float32)
    x[:10] = [127, 2.5, -2.5, 3.5, 0.5, -0.5, 1.5, -1.5, -127, 126.5]
    even = orc.quantize_q8_0(x, half_even=True)
    away = orc.quantize_q8_0(x, half_even=False)
    assert np.array_equal(even, _q8_block(0x3C00, [127, 2, -2, 4, 0, 0, 2, -2, -127, 126] + [0] * 22))
    assert np.array_equal(away, _q8_block(0x3C00, [127, 3, -3, 4, 1, -1, 2, -2, -127, 127] + [0] * 22))


def test_q8_quantize_power_of_two_scales(orc):
    """max|x| = 127 * 2^s gives d = 2^s exactly, so q = round(x / 2^s) and
    d's f16 bits are fixed; integers and integer + 1/2 over many scales."""
    rng = np.random.default_rng(5)
    for s in (-20, -7, 0, 3, 9):
        k = rng.integers(-127, 128, size=32).astype(np.float64)
        k[0] = 127
        k[1:8] += 0.5 * np.sign(rng.standard_normal(7))
        k = np.clip(k, -127, 127)
        x = (k * 2.0 ** s).astype(np.float32)
        for he in (True, False):
            got = orc.quantize_q8_0(x, half_even=he)
            q = np.rint(k) if he else np.sign(k) * np.floor(np.abs(k) + 0.5)
            dbits = int(np.array([2.0 ** s], np.float16).view(np.uint16)[0])
            assert np.array_equal(got, _q8_block(dbits, q.astype(int).tolist())), (s, he)


def test_q8_quantize_zero_and_underflowing_scale(orc):
    x = np.zeros(64, np.float32)
    # second block: d = 2^-40 underflows f16 (stored as 0) while q uses the f32 d
    x[32:] = (np.arange(32) - 16).astype(np.float32) * np.float32(2.0 ** -40)
    x[32] = np.float32(127 * 2.0 ** -40)
    got = orc.quantize_q8_0(x)
    assert np.array_equal(got[:34], np.zeros(34, np.uint8))
    qs = [127] + list(range(-15, 16))
    assert np.array_equal(got[34:], _q8_block(0, qs))


def test_q8_actq_reference_fixture_closed_form(orc):
    """The fixture of ops.rs:1212-1245 (rows d=1 q=[1,2,0..], d=2 q=[1,0..];
    x = 1..32).  d = 32/127, q1 = round(1/d) = 4, q2 = 8, f16(d) =
    0.251953125, so y = [20 * f16(d), 2 * 4 * f16(d)] exactly; the
    reference's own bar is 1 % of the f32 result [5, 2]."""
    w = np.concatenate([_q8_block(0x3C00, [1, 2] + [0] * 30), _q8_block(0x4000, [1] + [0] * 31)])
    x = np.arange(1, 33, dtype=np.float32)
    for he in (True, False):
        y = orc.matvec_q8_0_actq(w, 32, 2, x, half_even=he)
        assert y.tolist() == [5.0390625, 2.015625]
        assert abs(y[0] - 5.0) / 5.0 < 0.01 and abs(y[1] - 2.0) / 2.0 < 0.01


def test_q8_actq_matches_integer_brute_force(orc):
    """Block sums recomputed in exact integer arithmetic from the quantized
    bytes (float64 scaling): catches index / sign / scale slips in the dot."""
    n_in, n_out = 256, 9
    w = orc.gen_weight(Q8_0, 11, n_out, n_in)
    x = orc.gen_normal(12, n_in)
    xq = orc.quantize_q8_0(x).reshape(-1, 34)
    wq = w.reshape(n_out, -1, 34)
    f16 = lambda b: b[..., :2].copy().view(np.float16)[..., 0].astype(np.float64)
    dots = (wq[..., 2:].view(np.int8).astype(np.int64) * xq[None, :, 2:].view(np.int8)).sum(-1)
    ref = (f16(wq) * f16(xq)[None, :] * dots).sum(-1)
    y = orc.matvec_q8_0_actq(w, n_in, n_out, x)
    assert np.allclose(y, ref, rtol=1e-5, atol=1e-6 * np.abs(ref).max())
    # and it stays within the activation rounding of the f32 path
    y32 = orc.matvec(Q8_0, w, n_in, n_out, x)
    assert np.linalg.norm(y - y32) / np.linalg.norm(y32) < 2e-2
