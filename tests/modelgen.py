"""Seeded random-init models built on the host with the oracle's block
generator, so that the CPU oracle and the GPU see byte-identical weights."""
import numpy as np

F32, Q8_0, Q4_K, Q5_K, Q6_K = 0, 8, 12, 13, 14

TINY = dict(n_layer=2, n_embd=256, n_head=4, n_head_kv=2, head_dim=64, n_ff=512, vocab=512,
            rope_dim=64, ctx=96, rms_eps=1e-6, freq_base=10000.0)
# GQA with 5 query heads per KV head and head_dim 128, like the 32B shape
GQA5 = dict(n_layer=2, n_embd=1280, n_head=10, n_head_kv=2, head_dim=128, n_ff=1024,
            vocab=1000, rope_dim=128, ctx=160, rms_eps=1e-6, freq_base=1e6)
# head_dim 256 with 8 query heads per KV head: the split kernel's lane
# groups (8 at head_dim 256) each take one query head
HD256R8 = dict(n_layer=2, n_embd=512, n_head=8, n_head_kv=1, head_dim=256, n_ff=512, vocab=512,
               rope_dim=256, ctx=96, rms_eps=1e-6, freq_base=1e4)
# o and down with K = 2048 over few output tiles: the prompt block splits
# their K across workgroups and adds the slices in the fused reduce + RMSNorm
KSPLIT = dict(n_layer=2, n_embd=512, n_head=16, n_head_kv=2, head_dim=128, n_ff=2048,
              vocab=1000, rope_dim=128, ctx=160, rms_eps=1e-6, freq_base=1e6)

Q4_K_M = dict(attn_q=Q4_K, attn_k=Q4_K, attn_v=Q6_K, attn_output=Q4_K, ffn_gate=Q4_K,
              ffn_up=Q4_K, ffn_down=Q6_K, output=Q6_K, token_embd=Q4_K)
ALL_Q8_0 = {k: Q8_0 for k in Q4_K_M}
Q5_K_M = dict(Q4_K_M, attn_q=Q5_K, attn_k=Q5_K, attn_output=Q5_K, ffn_gate=Q5_K, ffn_up=Q5_K)


def shapes(cfg):
    E, qd, kvd, ff = cfg["n_embd"], cfg["n_head"] * cfg["head_dim"], \
        cfg["n_head_kv"] * cfg["head_dim"], cfg["n_ff"]
    return dict(attn_q=(E, qd), attn_k=(E, kvd), attn_v=(E, kvd), attn_output=(qd, E),
                ffn_gate=(E, ff), ffn_up=(E, ff), ffn_down=(ff, E))


def host_model(orc, cfg, seed=1, mix=None, mode=1, d_lo=2e-4, d_hi=2e-3, biases=True):
    """weights: name -> (type, array) in the oracle's naming (blk.{l}.{name})."""
    mix = dict(Q4_K_M, **(mix or {}))
    w = {}
    for l in range(cfg["n_layer"]):
        for i, (name, (n_in, n_out)) in enumerate(shapes(cfg).items()):
            t = mix[name]
            w[f"blk.{l}.{name}"] = (t, orc.gen_weight(t, seed * 1000 + l * 16 + i, n_out, n_in,
                                                     mode=mode, d_lo=d_lo, d_hi=d_hi))
        w[f"blk.{l}.attn_norm"] = (F32, orc.gen_uniform(seed * 77 + 4 * l, cfg["n_embd"], 0.9, 1.1))
        w[f"blk.{l}.ffn_norm"] = (F32, orc.gen_uniform(seed * 77 + 4 * l + 1, cfg["n_embd"], 0.9, 1.1))
        if biases:
            sh = shapes(cfg)
            w[f"blk.{l}.bq"] = (F32, orc.gen_uniform(seed * 91 + 4 * l, sh["attn_q"][1], -0.1, 0.1))
            w[f"blk.{l}.bk"] = (F32, orc.gen_uniform(seed * 91 + 4 * l + 1, sh["attn_k"][1], -0.1, 0.1))
            w[f"blk.{l}.bv"] = (F32, orc.gen_uniform(seed * 91 + 4 * l + 2, sh["attn_v"][1], -0.1, 0.1))
    w["token_embd"] = (mix["token_embd"], orc.gen_weight(mix["token_embd"], seed * 5 + 1,
                                                          cfg["vocab"], cfg["n_embd"], mode=mode,
                                                          d_lo=d_lo * 20, d_hi=d_hi * 20))
    w["output"] = (mix["output"], orc.gen_weight(mix["output"], seed * 5 + 2, cfg["vocab"],
                                                  cfg["n_embd"], mode=mode, d_lo=d_lo, d_hi=d_hi))
    w["output_norm"] = (F32, orc.gen_uniform(seed * 5 + 3, cfg["n_embd"], 0.9, 1.1))
    return w


def gpu_model(lrs, ctx, cfg, w):
    """Uploads a host model through the C ABI (the drop-in path)."""
    from llama_rs_amd.model import ResidentForward

    layers = []
    for l in range(cfg["n_layer"]):
        L = {}
        for name, (n_in, n_out) in shapes(cfg).items():
            t, arr = w[f"blk.{l}.{name}"]
            L[name] = lrs.Weight.upload(ctx, t, arr, n_in, n_out)
        for name in ("attn_norm", "ffn_norm", "bq", "bk", "bv"):
            if f"blk.{l}.{name}" in w:
                L[name] = w[f"blk.{l}.{name}"][1]
        layers.append(L)
    te, ta = w["token_embd"]
    emb = lrs.Weight.upload(ctx, te, ta, cfg["n_embd"], cfg["vocab"])
    ot, oa = w["output"]
    out = lrs.Weight.upload(ctx, ot, oa, cfg["n_embd"], cfg["vocab"])
    return ResidentForward(ctx, cfg, layers, emb, w["output_norm"][1], out)


def attn_splits(n_kv):
    """position splits of the decode attention per KV head (attention.hip
    attn_splits): 256 / n_kv workgroups, at least 1 and at most 40"""
    return max(1, min(40, 256 // n_kv))


def split_block_checks(n_kv, rounds=2):
    """cache lengths at which the decode attention's splits (split s owns the
    16-position blocks s, s + S, s + 2S, ...) first own 1 .. rounds + 1 blocks:
    16 S r and 16 S r + 1 for r = 1 .. rounds, plus 1, 16 and 17"""
    S = attn_splits(n_kv)
    out = [1, 16, 17]
    for r in range(1, rounds + 1):
        out += [16 * S * r, 16 * S * r + 1]
    return tuple(out)


def oracle_greedy(model, prompt, n_gen):
    """Model::generate with greedy sampling: forward(prompt), then one token
    at a time (generate.rs:13-43)."""
    toks = []
    logits = model.forward(np.asarray(prompt, np.uint32))
    nxt = int(np.argmax(logits))  # first index of the max, like ops::argmax
    for _ in range(n_gen):
        toks.append(nxt)
        if len(toks) == n_gen:
            break
        logits = model.forward(np.asarray([nxt], np.uint32))
        nxt = int(np.argmax(logits))
    return toks


# ---------------------------------------------------------------------------
# hybrid attention + gated delta-net (qwen35-shaped) models
# ---------------------------------------------------------------------------
# layers 0-2 delta net, layer 3 full attention; 4 value heads over 2 key heads
# (the modulo GQA mapping), partial RoPE
HY_TINY = dict(n_layer=4, n_embd=256, n_head=4, n_head_kv=2, head_dim=64, n_ff=512, vocab=512,
               rope_dim=32, ctx=64, rms_eps=1e-6, freq_base=1e7, full_attn_interval=4,
               dn_k_heads=2, dn_v_heads=4, dn_state=64, dn_conv=4)
# the config-4 head shapes (24/4 x 256 attention -> GQA 6, d_state 128) at a
# small width
HY_MID = dict(n_layer=4, n_embd=512, n_head=6, n_head_kv=1, head_dim=256, n_ff=768, vocab=1024,
              rope_dim=64, ctx=64, rms_eps=1e-6, freq_base=1e7, full_attn_interval=2,
              dn_k_heads=2, dn_v_heads=2, dn_state=128, dn_conv=4)
# K = 2048 for o (8 x 256), ssm_out (16 x 128 state columns) and down: the
# prompt block's K-split GEMMs and the fused reduce + RMSNorm, including the
# f32 normalised rows a delta-net layer reads
HY_KS = dict(HY_MID, n_head=8, n_ff=2048, dn_k_heads=4, dn_v_heads=16)

HY_Q4_K_M = dict(Q4_K_M, ssm_qkv=Q4_K, ssm_gate=Q4_K, ssm_out=Q4_K)


def hy_conv_dim(cfg):
    return (2 * cfg["dn_k_heads"] + cfg["dn_v_heads"]) * cfg["dn_state"]


def hy_is_full(cfg, l):
    return (l + 1) % cfg["full_attn_interval"] == 0


def hybrid_shapes(cfg, l):
    """(n_in, n_out) of the quantized matrices of layer l."""
    E, ff = cfg["n_embd"], cfg["n_ff"]
    sh = dict(ffn_gate=(E, ff), ffn_up=(E, ff), ffn_down=(ff, E))
    if hy_is_full(cfg, l):
        qd, kvd = cfg["n_head"] * cfg["head_dim"], cfg["n_head_kv"] * cfg["head_dim"]
        sh.update(attn_q=(E, 2 * qd), attn_k=(E, kvd), attn_v=(E, kvd), attn_output=(qd, E))
    else:
        vd = cfg["dn_v_heads"] * cfg["dn_state"]
        sh.update(ssm_qkv=(E, hy_conv_dim(cfg)), ssm_gate=(E, vd), ssm_out=(vd, E))
    return sh


def hybrid_f32_shapes(cfg, l):
    """element counts of the f32 vectors of layer l and their uniform ranges."""
    E = cfg["n_embd"]
    sh = dict(attn_norm=(E, 0.9, 1.1), post_norm=(E, 0.9, 1.1))
    if hy_is_full(cfg, l):
        sh.update(q_norm=(cfg["head_dim"], 0.9, 1.1), k_norm=(cfg["head_dim"], 0.9, 1.1))
    else:
        nv, r = cfg["dn_v_heads"], 1.7 / np.sqrt(E)
        sh.update(ssm_alpha=(nv * E, -r, r), ssm_beta=(nv * E, -r, r), ssm_a=(nv, -1.0, -0.1),
                  ssm_dt=(nv, -1.0, 1.0), ssm_conv=(hy_conv_dim(cfg) * cfg["dn_conv"], -0.5, 0.5),
                  ssm_norm=(cfg["dn_state"], 0.9, 1.1))
    return sh


def hybrid_host_model(orc, cfg, seed=1, mix=None, mode=1, d_lo=2e-4, d_hi=2e-3):
    mix = dict(HY_Q4_K_M, **(mix or {}))
    w = {}
    for l in range(cfg["n_layer"]):
        for i, (name, (n_in, n_out)) in enumerate(sorted(hybrid_shapes(cfg, l).items())):
            t = mix[name]
            w[f"blk.{l}.{name}"] = (t, orc.gen_weight(t, seed * 1000 + l * 32 + i, n_out, n_in,
                                                     mode=mode, d_lo=d_lo, d_hi=d_hi))
        for i, (name, (n, lo, hi)) in enumerate(sorted(hybrid_f32_shapes(cfg, l).items())):
            w[f"blk.{l}.{name}"] = (F32, orc.gen_uniform(seed * 77 + 32 * l + i, n, lo, hi))
    w["token_embd"] = (mix["token_embd"], orc.gen_weight(mix["token_embd"], seed * 5 + 1,
                                                          cfg["vocab"], cfg["n_embd"], mode=mode,
                                                          d_lo=d_lo * 20, d_hi=d_hi * 20))
    w["output"] = (mix["output"], orc.gen_weight(mix["output"], seed * 5 + 2, cfg["vocab"],
                                                  cfg["n_embd"], mode=mode, d_lo=d_lo, d_hi=d_hi))
    w["output_norm"] = (F32, orc.gen_uniform(seed * 5 + 3, cfg["n_embd"], 0.9, 1.1))
    return w


def hybrid_device_model(lrs, ctx, orc, cfg, seed=1, mix=None, mode=1, d_lo=2e-4, d_hi=2e-3):
    """The weights of hybrid_host_model(orc, cfg, seed, mix, mode, d_lo, d_hi),
    the quantized ones generated on the GPU (the device generator writes the
    oracle generator's bytes; test_device_generator_matches_host_generator)
    and downloaded for the oracle.  Returns (host weight dict, GPU model) on
    the same bytes; much faster than host generation at full width."""
    from llama_rs_amd.model import HybridForward

    mix = dict(HY_Q4_K_M, **(mix or {}))
    w, layers = {}, []
    for l in range(cfg["n_layer"]):
        L = {}
        for i, (name, (n_in, n_out)) in enumerate(sorted(hybrid_shapes(cfg, l).items())):
            t = mix[name]
            L[name] = lrs.Weight.generate(ctx, t, seed * 1000 + l * 32 + i, n_in, n_out,
                                          mode=mode, d_lo=d_lo, d_hi=d_hi)
            w[f"blk.{l}.{name}"] = (t, L[name].download())
        for i, (name, (n, lo, hi)) in enumerate(sorted(hybrid_f32_shapes(cfg, l).items())):
            w[f"blk.{l}.{name}"] = (F32, orc.gen_uniform(seed * 77 + 32 * l + i, n, lo, hi))
            L[name] = w[f"blk.{l}.{name}"][1]
        layers.append(L)
    te, ot = mix["token_embd"], mix["output"]
    emb = lrs.Weight.generate(ctx, te, seed * 5 + 1, cfg["n_embd"], cfg["vocab"], mode=mode,
                              d_lo=d_lo * 20, d_hi=d_hi * 20)
    out = lrs.Weight.generate(ctx, ot, seed * 5 + 2, cfg["n_embd"], cfg["vocab"], mode=mode,
                              d_lo=d_lo, d_hi=d_hi)
    w["token_embd"] = (te, emb.download())
    w["output"] = (ot, out.download())
    w["output_norm"] = (F32, orc.gen_uniform(seed * 5 + 3, cfg["n_embd"], 0.9, 1.1))
    return w, HybridForward(ctx, cfg, layers, emb, w["output_norm"][1], out)


def gpu_hybrid_model(lrs, ctx, cfg, w):
    """Uploads a host hybrid model through the C ABI."""
    from llama_rs_amd.model import HybridForward

    layers = []
    for l in range(cfg["n_layer"]):
        L = {}
        for name, (n_in, n_out) in hybrid_shapes(cfg, l).items():
            t, arr = w[f"blk.{l}.{name}"]
            L[name] = lrs.Weight.upload(ctx, t, arr, n_in, n_out)
        for name in hybrid_f32_shapes(cfg, l):
            L[name] = w[f"blk.{l}.{name}"][1]
        layers.append(L)
    te, ta = w["token_embd"]
    emb = lrs.Weight.upload(ctx, te, ta, cfg["n_embd"], cfg["vocab"])
    ot, oa = w["output"]
    out = lrs.Weight.upload(ctx, ot, oa, cfg["n_embd"], cfg["vocab"])
    return HybridForward(ctx, cfg, layers, emb, w["output_norm"][1], out)


def write_model_gguf(path, cfg, w):
    """Writes a host model (dense or hybrid weight dict) as a GGUF file with
    the tensor names and metadata the loader reads (gpu.rs, config.rs)."""
    from llama_rs_amd.gguf import GGUF_NAMES, model_kv, vector_dims, write_gguf

    hybrid = "full_attn_interval" in cfg
    tensors = []
    for key, (t, arr) in w.items():
        if key.startswith("blk."):
            _, l, name = key.split(".", 2)
            gname = f"blk.{l}.{GGUF_NAMES[name]}"
        else:
            gname = key + ".weight"
            name = key
        if t == F32:
            dims = vector_dims(cfg, name, arr.size)
        else:
            if key.startswith("blk."):
                sh = hybrid_shapes(cfg, int(l)) if hybrid else shapes(cfg)
                n_in, n_out = sh[name]
            else:
                n_in, n_out = cfg["n_embd"], cfg["vocab"]
            dims = [n_in, n_out]
        tensors.append((gname, t, dims, np.ascontiguousarray(arr).tobytes()))
    write_gguf(path, model_kv(cfg, "qwen35" if hybrid else "qwen2"), tensors)
