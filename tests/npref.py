"""Independent numpy restatements used to pin the C oracle.

These are written from the GGUF block layouts element-by-element (vectorised
index arithmetic per output element), not by transcribing the loop structure
of crates/ggml-cpu/src/dequant.rs, so that a wrong nibble, bit pair or scale
index in either implementation shows up as a mismatch.  float32 numpy
arithmetic rounds after every operation (no FMA), which is what the reference's
Rust code does, so the dequant comparisons are bit-exact.
"""
from __future__ import annotations

import numpy as np

F32, F16, Q4_0, Q8_0, Q4_K, Q5_K, Q6_K = 0, 1, 2, 8, 12, 13, 14
TYPE_SIZE = {F32: 4, F16: 2, Q4_0: 18, Q8_0: 34, Q4_K: 144, Q5_K: 176, Q6_K: 210}


def _f16(b: np.ndarray, off: int) -> np.ndarray:
    """little-endian binary16 at byte offset `off` of each block row -> float32"""
    raw = (b[:, off].astype(np.uint16) | (b[:, off + 1].astype(np.uint16) << 8))
    return raw.view(np.float16).astype(np.float32)


def kquant_scales(s12: np.ndarray):
    """(n,12) packed bytes -> (sc, m) each (n,8) uint8: bytes 0-3 hold sc[0..3]
    in their low 6 bits and bits 4-5 of sc[4..7] on top; bytes 4-7 the same for
    m; bytes 8-11 hold the low nibbles of sc[4..7] (low) and m[4..7] (high)."""
    s12 = s12.astype(np.uint16)
    sc = np.zeros((s12.shape[0], 8), np.uint16)
    m = np.zeros_like(sc)
    sc[:, :4] = s12[:, 0:4] & 0x3F
    m[:, :4] = s12[:, 4:8] & 0x3F
    sc[:, 4:] = (s12[:, 8:12] & 0x0F) | ((s12[:, 0:4] >> 6) << 4)
    m[:, 4:] = (s12[:, 8:12] >> 4) | ((s12[:, 4:8] >> 6) << 4)
    return sc.astype(np.uint8), m.astype(np.uint8)


def dequant(t: int, data: np.ndarray) -> np.ndarray:
    data = np.ascontiguousarray(data)
    if data.dtype != np.uint8:
        data = data.view(np.uint8)
    ts = TYPE_SIZE[t]
    assert data.size % ts == 0
    b = data.reshape(-1, ts)
    n = b.shape[0]
    if t == F32:
        return b.reshape(-1).view(np.float32).copy()
    if t == F16:
        return b.reshape(-1).view(np.float16).astype(np.float32)
    if t == Q8_0:
        d = _f16(b, 0)[:, None]
        q = b[:, 2:34].view(np.int8).astype(np.float32)
        return (q * d).reshape(-1)
    if t == Q4_0:
        d = _f16(b, 0)[:, None]
        e = np.arange(32)
        byte = b[:, 2 + (e % 16)]
        nib = np.where(e < 16, byte & 0x0F, byte >> 4).astype(np.int32) - 8
        return (nib.astype(np.float32) * d).reshape(-1)
    if t in (Q4_K, Q5_K):
        d = _f16(b, 0)[:, None]
        dmin = _f16(b, 2)[:, None]
        sc, m = kquant_scales(b[:, 4:16])
        qs_off = 16 if t == Q4_K else 48
        e = np.arange(256)
        grp, within = e // 64, e % 64
        sub = 2 * grp + (within >= 32)
        l = within % 32
        byte = b[:, qs_off + 32 * grp + l]
        q = np.where(within < 32, byte & 0x0F, byte >> 4).astype(np.int32)
        if t == Q5_K:
            qh = b[:, 16 + l]
            q = q + 16 * ((qh >> sub) & 1).astype(np.int32)
        dsc = d * sc[:, sub].astype(np.float32)
        dm = dmin * m[:, sub].astype(np.float32)
        return (dsc * q.astype(np.float32) - dm).reshape(-1)
    if t == Q6_K:
        d = _f16(b, 208)[:, None]
        scales = b[:, 192:208].view(np.int8).astype(np.float32)
        e = np.arange(256)
        half, within = e // 128, e % 128
        quarter, l = within // 32, within % 32
        qlb = b[:, 64 * half + l + 32 * (quarter % 2)]
        lo = np.where(quarter < 2, qlb & 0x0F, qlb >> 4).astype(np.int32)
        hi = ((b[:, 128 + 32 * half + l] >> (2 * quarter)) & 3).astype(np.int32)
        q = (lo | (hi << 4)) - 32
        s = scales[:, 8 * half + l // 16 + 2 * quarter]
        return ((d * s) * q.astype(np.float32)).reshape(-1)
    raise ValueError(t)


def rms_forward64(cfg: dict, weights: dict, tokens, kv_f16: bool):
    """float64 restatement of the dense forward (model.rs:99-266), computed with
    numpy's pairwise/BLAS sums: pins the structure of the C forward (op order,
    residual wiring, GQA head mapping, RoPE pairing, causal mask) to ~1e-5."""
    c = cfg
    E, H, HKV, HD = c["n_embd"], c["n_head"], c["n_head_kv"], c["head_dim"]
    KV = HKV * HD

    def W(name, n_in, n_out):
        t, arr = weights[name]
        return dequant(t, arr).astype(np.float64).reshape(n_out, n_in)

    def vec(name):
        t, arr = weights[name]
        return dequant(t, arr).astype(np.float64)

    def norm(x, w):
        return x / np.sqrt((x * x).mean(-1, keepdims=True) + c["rms_eps"]) * w

    def rope(x, nh, pos0):
        n = x.shape[0]
        x = x.reshape(n, nh, HD).copy()
        i = np.arange(c["rope_dim"] // 2)
        freq = np.float64(c["freq_base"]) ** (-2.0 * i / c["rope_dim"])
        pos = (pos0 + np.arange(n))[:, None].astype(np.float64)
        th = pos * freq[None, :]
        cs, sn = np.cos(th)[:, None, :], np.sin(th)[:, None, :]
        a = x[:, :, 0:c["rope_dim"]:2].copy()
        b2 = x[:, :, 1:c["rope_dim"]:2].copy()
        x[:, :, 0:c["rope_dim"]:2] = a * cs - b2 * sn
        x[:, :, 1:c["rope_dim"]:2] = a * sn + b2 * cs
        return x.reshape(n, nh * HD)

    tokens = np.asarray(tokens)
    n_layer = c["n_layer"]
    emb = W("token_embd", E, c["vocab"])
    x = emb[tokens]
    kcache = [np.zeros((0, KV)) for _ in range(n_layer)]
    vcache = [np.zeros((0, KV)) for _ in range(n_layer)]
    out_logits = []
    for li in range(n_layer):
        p = f"blk.{li}."
        h = norm(x, vec(p + "attn_norm"))
        q = h @ W(p + "attn_q", E, H * HD).T
        k = h @ W(p + "attn_k", E, KV).T
        v = h @ W(p + "attn_v", E, KV).T
        for nm, arr in (("bq", q), ("bk", k), ("bv", v)):
            if weights.get(p + nm) is not None:
                arr += vec(p + nm)
        q = rope(q, H, 0)
        k = rope(k, HKV, 0)
        if kv_f16:
            k = k.astype(np.float32).astype(np.float16).astype(np.float64)
            v = v.astype(np.float32).astype(np.float16).astype(np.float64)
        n = x.shape[0]
        att = np.zeros((n, H * HD))
        rep = H // HKV
        for t in range(n):
            for hh in range(H):
                kh = hh // rep
                qv = q[t, hh * HD:(hh + 1) * HD]
                ks = k[:t + 1, kh * HD:(kh + 1) * HD]
                vs = v[:t + 1, kh * HD:(kh + 1) * HD]
                s = ks @ qv / np.sqrt(HD)
                s = np.exp(s - s.max())
                s /= s.sum()
                att[t, hh * HD:(hh + 1) * HD] = s @ vs
        x = x + att @ W(p + "attn_output", H * HD, E).T
        h = norm(x, vec(p + "ffn_norm"))
        g = h @ W(p + "ffn_gate", E, c["n_ff"]).T
        u = h @ W(p + "ffn_up", E, c["n_ff"]).T
        a = g / (1.0 + np.exp(-g)) * u
        x = x + a @ W(p + "ffn_down", c["n_ff"], E).T
    h = norm(x, vec("output_norm"))
    return h @ W("output", E, c["vocab"]).T


def hybrid_forward64(c, weights, tokens, kv_f16=True):
    """float64 restatement of the hybrid (qwen35) decode, one token at a time:
    full attention when (l+1) % full_attn_interval == 0 (config.rs:25-35),
    else the gated delta net of plano_delta (resident_forward.rs:2252-2470).
    Written from the formulas (delta rule as S <- a S + beta (v - a S k) k^T on
    a row-major S[v][k] matrix) rather than from the oracle's loops.  Returns
    the logits of every token [n_tok][vocab]."""
    E, H, HKV, HD = c["n_embd"], c["n_head"], c["n_head_kv"], c["head_dim"]
    NK, NV, D, W = c["dn_k_heads"], c["dn_v_heads"], c["dn_state"], c["dn_conv"]
    eps = c["rms_eps"]

    def mat(name, n_in, n_out):
        t, arr = weights[name]
        return dequant(t, arr).astype(np.float64).reshape(n_out, n_in)

    def vec(name):
        t, arr = weights[name]
        return dequant(t, arr).astype(np.float64)

    def rms(x, w):
        return x / np.sqrt((x * x).mean(-1, keepdims=True) + eps) * w

    def silu(v):
        return v / (1.0 + np.exp(-v))

    half = c["rope_dim"] // 2
    inv_freq = 1.0 / np.float64(c["freq_base"]) ** (2.0 * np.arange(half) / c["rope_dim"])

    def rope(heads, pos):  # heads [n, HD]; adjacent pairs of the first rope_dim dims
        out = heads.copy()
        th = pos * inv_freq
        a, b = heads[:, 0:2 * half:2], heads[:, 1:2 * half:2]
        out[:, 0:2 * half:2] = a * np.cos(th) - b * np.sin(th)
        out[:, 1:2 * half:2] = a * np.sin(th) + b * np.cos(th)
        return out

    full = [(l + 1) % c["full_attn_interval"] == 0 for l in range(c["n_layer"])]
    kcache = {l: [] for l in range(c["n_layer"]) if full[l]}
    vcache = {l: [] for l in range(c["n_layer"]) if full[l]}
    S = {l: np.zeros((NV, D, D)) for l in range(c["n_layer"]) if not full[l]}
    CD = (2 * NK + NV) * D
    hist = {l: np.zeros((W - 1, CD)) for l in range(c["n_layer"]) if not full[l]}
    emb = mat("token_embd", E, c["vocab"])
    logits = []
    for pos, tok in enumerate(np.asarray(tokens)):
        x = emb[tok].copy()
        for l in range(c["n_layer"]):
            p = f"blk.{l}."
            h = rms(x, vec(p + "attn_norm"))
            if full[l]:
                qg = (mat(p + "attn_q", E, 2 * H * HD) @ h).reshape(H, 2, HD)
                q, gate = qg[:, 0, :], qg[:, 1, :]
                k = (mat(p + "attn_k", E, HKV * HD) @ h).reshape(HKV, HD)
                v = (mat(p + "attn_v", E, HKV * HD) @ h).reshape(HKV, HD)
                q = rope(rms(q, vec(p + "q_norm")), pos)
                k = rope(rms(k, vec(p + "k_norm")), pos)
                if kv_f16:
                    k = k.astype(np.float32).astype(np.float16).astype(np.float64)
                    v = v.astype(np.float32).astype(np.float16).astype(np.float64)
                kcache[l].append(k)
                vcache[l].append(v)
                K, V = np.stack(kcache[l]), np.stack(vcache[l])  # [t, HKV, HD]
                att = np.zeros((H, HD))
                for hh in range(H):
                    kh = hh // (H // HKV)
                    s = K[:, kh, :] @ q[hh] / np.sqrt(HD)
                    s = np.exp(s - s.max())
                    att[hh] = (s / s.sum()) @ V[:, kh, :]
                att = att / (1.0 + np.exp(-gate))
                o = mat(p + "attn_output", H * HD, E) @ att.reshape(-1)
            else:
                qkv = mat(p + "ssm_qkv", E, CD) @ h
                z = (mat(p + "ssm_gate", E, NV * D) @ h).reshape(NV, D)
                ker = vec(p + "ssm_conv").reshape(CD, W)
                win = np.vstack([hist[l], qkv[None, :]])  # oldest first, [W, CD]
                conv = silu((win * ker.T).sum(0))
                hist[l] = win[1:]
                q = conv[:NK * D].reshape(NK, D)
                k = conv[NK * D:2 * NK * D].reshape(NK, D)
                v = conv[2 * NK * D:].reshape(NV, D)
                q = q / np.sqrt((q * q).sum(-1, keepdims=True) + eps)
                k = k / np.sqrt((k * k).sum(-1, keepdims=True) + eps)
                alpha = vec(p + "ssm_alpha").reshape(NV, E) @ h
                beta = 1.0 / (1.0 + np.exp(-(vec(p + "ssm_beta").reshape(NV, E) @ h)))
                a = np.exp(vec(p + "ssm_a") * np.log1p(np.exp(alpha + vec(p + "ssm_dt"))))
                y = np.zeros((NV, D))
                for hh in range(NV):
                    kk, qq = k[hh % NK], q[hh % NK]
                    Sh = a[hh] * S[l][hh]                     # S[v, k]
                    Sh = Sh + beta[hh] * np.outer(v[hh] - Sh @ kk, kk)
                    S[l][hh] = Sh
                    y[hh] = Sh @ qq / np.sqrt(D)
                y = rms(y, vec(p + "ssm_norm")) * silu(z)
                o = mat(p + "ssm_out", NV * D, E) @ y.reshape(-1)
            x = x + o
            h = rms(x, vec(p + "post_norm"))
            g = mat(p + "ffn_gate", E, c["n_ff"]) @ h
            u = mat(p + "ffn_up", E, c["n_ff"]) @ h
            x = x + mat(p + "ffn_down", c["n_ff"], E) @ (silu(g) * u)
        logits.append(mat("output", E, c["vocab"]) @ rms(x, vec("output_norm")))
    return np.stack(logits)
