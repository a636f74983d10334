"""ResidentForward — host mirror of llama_model::GpuResidentDecode
(crates/llama-model/src/gpu.rs:379-455) over liblrs.so's model entry points.

Methods keep the reference's names and meaning: ``decode(token, pos)`` returns
the logits of one token at absolute position ``pos`` (the KV cache then holds
``pos + 1`` positions), ``decode_batch(tokens, pos0)`` the logits of the last
of a block, ``batch_size()``, ``reset()``.  ``decode_greedy`` and
``generate_greedy`` keep the argmax on the device (the temperature-0 path of
gerar_streaming_residente, gpu.rs:609-666).  Failures raise ModelError.
"""
from __future__ import annotations

import ctypes as C

import numpy as np

from . import Context, ModelError, Weight, check, lib, Q4_K, Q6_K

_u32p = C.POINTER(C.c_uint32)
_f32p = C.POINTER(C.c_float)


class LrsConfig(C.Structure):
    _fields_ = [(n, C.c_uint32) for n in
                ("n_layer", "n_embd", "n_head", "n_head_kv", "head_dim", "n_ff", "vocab",
                 "rope_dim", "ctx")] + [("rms_eps", C.c_float), ("freq_base", C.c_float)]


class LrsLayer(C.Structure):
    _fields_ = [(n, C.c_void_p) for n in
                ("attn_q", "attn_k", "attn_v", "attn_output", "ffn_gate", "ffn_up", "ffn_down",
                 "attn_norm", "ffn_norm", "bq", "bk", "bv")]


class LrsHybridConfig(C.Structure):
    _fields_ = [("base", LrsConfig)] + [(n, C.c_uint32) for n in
                                        ("full_attn_interval", "dn_k_heads", "dn_v_heads",
                                         "dn_state", "dn_conv")]


HYBRID_WEIGHTS = ("ffn_gate", "ffn_up", "ffn_down")
HYBRID_LAYER_FIELDS = (("ffn_gate", "w"), ("ffn_up", "w"), ("ffn_down", "w"),
                       ("attn_norm", "f"), ("post_norm", "f"),
                       ("attn_q", "w"), ("attn_k", "w"), ("attn_v", "w"), ("attn_output", "w"),
                       ("q_norm", "f"), ("k_norm", "f"),
                       ("ssm_qkv", "w"), ("ssm_gate", "w"), ("ssm_out", "w"),
                       ("ssm_alpha", "f"), ("ssm_beta", "f"), ("ssm_a", "f"), ("ssm_dt", "f"),
                       ("ssm_conv", "f"), ("ssm_norm", "f"))


class LrsHybridLayer(C.Structure):
    _fields_ = [(n, C.c_void_p) for n, _ in HYBRID_LAYER_FIELDS]


def _bind():
    vp = C.c_void_p
    sig = {
        "lrs_model_create": (C.c_int, [vp, C.POINTER(LrsConfig), vp, vp, vp, vp, C.POINTER(vp)]),
        "lrs_hybrid_create": (C.c_int, [vp, C.POINTER(LrsHybridConfig), vp, vp, vp, vp,
                                        C.POINTER(vp)]),
        "lrs_model_destroy": (None, [vp]),
        "lrs_decode": (C.c_int, [vp, C.c_uint32, C.c_uint32, vp]),
        "lrs_decode_batch": (C.c_int, [vp, vp, C.c_uint32, C.c_uint32, vp]),
        "lrs_batch_size": (C.c_uint32, [vp]),
        "lrs_reset": (None, [vp]),
        "lrs_model_len": (C.c_uint32, [vp]),
        "lrs_decode_greedy": (C.c_int, [vp, C.c_uint32, C.c_uint32, _u32p]),
        "lrs_generate_greedy": (C.c_int, [vp, vp, C.c_uint32, C.c_uint32, C.c_uint32, vp]),
        "lrs_model_profile": (C.c_int, [vp, C.c_uint32, C.c_uint32, C.POINTER(C.c_float),
                                        C.POINTER(C.c_size_t)]),
        "lrs_model_bytes_per_token": (C.c_size_t, [vp]),
        "lrs_model_set_q8_rounding": (C.c_int, [vp, C.c_int]),
    }
    for name, (res, args) in sig.items():
        f = getattr(lib, name)
        f.restype = res
        f.argtypes = args


_bind()

CONFIG_KEYS = ("n_layer", "n_embd", "n_head", "n_head_kv", "head_dim", "n_ff", "vocab",
               "rope_dim", "ctx", "rms_eps", "freq_base")


def _f32(a):
    return None if a is None else np.ascontiguousarray(a, dtype=np.float32)


class ResidentForward:
    """The whole model resident on one GPU; one HIP graph per token."""

    def __init__(self, ctx: Context, cfg: dict, layers: list, token_embd: Weight,
                 output_norm, output: Weight):
        self.ctx, self.cfg = ctx, dict(cfg)
        c = LrsConfig(*[cfg[k] for k in CONFIG_KEYS])
        self._keep = [token_embd, output]
        arr = (LrsLayer * cfg["n_layer"])()
        for i, L in enumerate(layers):
            vecs = {k: _f32(L.get(k)) for k in ("attn_norm", "ffn_norm", "bq", "bk", "bv")}
            self._keep.append(vecs)
            self._keep.extend(L[k] for k in ("attn_q", "attn_k", "attn_v", "attn_output",
                                             "ffn_gate", "ffn_up", "ffn_down"))
            for k in ("attn_q", "attn_k", "attn_v", "attn_output", "ffn_gate", "ffn_up",
                      "ffn_down"):
                setattr(arr[i], k, L[k].h.value if isinstance(L[k].h, C.c_void_p) else L[k].h)
            for k, v in vecs.items():
                setattr(arr[i], k, None if v is None else v.ctypes.data)
        onorm = _f32(output_norm)
        self._keep.append(onorm)
        h = C.c_void_p()

        def wh(w):
            return w.h.value if isinstance(w.h, C.c_void_p) else w.h

        check(lib.lrs_model_create(ctx.h, C.byref(c), C.cast(arr, C.c_void_p), wh(token_embd),
                                   onorm.ctypes.data, wh(output), C.byref(h)))
        self.h = h
        self.vocab = cfg["vocab"]
        ctx._models.add(self)

    # --- GpuResidentDecode -------------------------------------------------
    def decode(self, token: int, pos: int) -> np.ndarray:
        out = np.empty(self.vocab, np.float32)
        check(lib.lrs_decode(self.h, int(token), int(pos), out.ctypes.data))
        return out

    def decode_batch(self, tokens, pos0: int) -> np.ndarray:
        t = np.ascontiguousarray(tokens, dtype=np.uint32)
        out = np.empty(self.vocab, np.float32)
        check(lib.lrs_decode_batch(self.h, t.ctypes.data, t.size, int(pos0), out.ctypes.data))
        return out

    def batch_size(self) -> int:
        return int(lib.lrs_batch_size(self.h))

    def reset(self) -> None:
        lib.lrs_reset(self.h)

    def __len__(self) -> int:
        return int(lib.lrs_model_len(self.h))

    def set_q8_rounding(self, on: bool) -> None:
        """Q8_0 weights multiply their input rounded to Q8_0 like the reference
        CPU forward (weights.rs:109-124), instead of the f32 activation."""
        check(lib.lrs_model_set_q8_rounding(self.h, int(bool(on))))

    # --- device-side greedy ------------------------------------------------
    def decode_greedy(self, token: int, pos: int) -> int:
        nxt = C.c_uint32()
        check(lib.lrs_decode_greedy(self.h, int(token), int(pos), C.byref(nxt)))
        return int(nxt.value)

    def generate_greedy(self, prompt, n_gen: int, pos0: int = 0) -> np.ndarray:
        p = np.ascontiguousarray(prompt, dtype=np.uint32)
        out = np.empty(n_gen, np.uint32)
        check(lib.lrs_generate_greedy(self.h, p.ctypes.data, p.size, int(pos0), int(n_gen),
                                      out.ctypes.data))
        return out

    OPS = {"qkv": 0, "attn": 1, "o": 2, "gateup": 3, "down": 4, "head": 5,
           "dn_proj": 6, "dn_step": 7, "dn_out": 8, "qk_prep": 9, "ffn": 10,
           "matvecs": 11}

    def profile(self, op: str, iters: int):
        """(mean us per launch, bytes per launch) of one fused op, outside the graph."""
        us, b = C.c_float(), C.c_size_t()
        check(lib.lrs_model_profile(self.h, self.OPS[op], int(iters), C.byref(us), C.byref(b)))
        return float(us.value), int(b.value)

    @property
    def bytes_per_token(self) -> int:
        return int(lib.lrs_model_bytes_per_token(self.h))

    def close(self) -> None:
        if getattr(self, "h", None) and self.ctx.h:
            lib.lrs_model_destroy(self.h)
        self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def _wh(w):
    return w.h.value if isinstance(w.h, C.c_void_p) else w.h


class HybridForward(ResidentForward):
    """Hybrid (qwen35) model: gated full attention every
    ``full_attn_interval``-th layer, gated delta net elsewhere.  Same decode
    interface; positions must continue the sequence (the recurrent state
    cannot be rewound) and ``reset()`` clears it."""

    def __init__(self, ctx: Context, cfg: dict, layers: list, token_embd: Weight,
                 output_norm, output: Weight):
        self.ctx, self.cfg = ctx, dict(cfg)
        base = LrsConfig(*[cfg[k] for k in CONFIG_KEYS])
        c = LrsHybridConfig(base, cfg["full_attn_interval"], cfg["dn_k_heads"],
                            cfg["dn_v_heads"], cfg["dn_state"], cfg["dn_conv"])
        self._keep = [token_embd, output]
        arr = (LrsHybridLayer * cfg["n_layer"])()
        for i, L in enumerate(layers):
            for name, kind in HYBRID_LAYER_FIELDS:
                v = L.get(name)
                if v is None:
                    continue
                if kind == "w":
                    self._keep.append(v)
                    setattr(arr[i], name, _wh(v))
                else:
                    a = _f32(v)
                    self._keep.append(a)
                    setattr(arr[i], name, a.ctypes.data)
        onorm = _f32(output_norm)
        self._keep.append(onorm)
        h = C.c_void_p()
        check(lib.lrs_hybrid_create(ctx.h, C.byref(c), C.cast(arr, C.c_void_p), _wh(token_embd),
                                    onorm.ctypes.data, _wh(output), C.byref(h)))
        self.h = h
        self.vocab = cfg["vocab"]
        ctx._models.add(self)


# ---------------------------------------------------------------------------
# synthetic random-init models generated on the device (no host copy)
# ---------------------------------------------------------------------------
QWEN25_32B = dict(n_layer=64, n_embd=5120, n_head=40, n_head_kv=8, head_dim=128, n_ff=27648,
                  vocab=152064, rope_dim=128, ctx=4096, rms_eps=1e-6, freq_base=1e6)
# Q4_K_M mix used for the benchmark: q,k,o,gate,up Q4_K; v,down Q6_K; head Q6_K
Q4_K_M_MIX = dict(attn_q=Q4_K, attn_k=Q4_K, attn_v=Q6_K, attn_output=Q4_K, ffn_gate=Q4_K,
                  ffn_up=Q4_K, ffn_down=Q6_K, output=Q6_K, token_embd=Q4_K)


def layer_shapes(cfg):
    E, qd, kvd, ff = cfg["n_embd"], cfg["n_head"] * cfg["head_dim"], \
        cfg["n_head_kv"] * cfg["head_dim"], cfg["n_ff"]
    return dict(attn_q=(E, qd), attn_k=(E, kvd), attn_v=(E, kvd), attn_output=(qd, E),
                ffn_gate=(E, ff), ffn_up=(E, ff), ffn_down=(ff, E))


def synthetic_model(ctx: Context, cfg: dict, seed: int = 1, mix: dict | None = None,
                    mode: int = 0, d_lo: float = 1e-3, d_hi: float = 1e-2,
                    biases: bool = True):
    """Random-init model of the given shape with weights generated on the GPU
    (seeded GGUF blocks), norm weights ~U[0.9, 1.1] and small q/k/v biases."""
    mix = dict(Q4_K_M_MIX, **(mix or {}))
    rng = np.random.default_rng(seed)
    shapes = layer_shapes(cfg)
    layers = []
    for l in range(cfg["n_layer"]):
        L = {}
        for i, (name, (n_in, n_out)) in enumerate(shapes.items()):
            L[name] = Weight.generate(ctx, mix[name], seed * 1000003 + l * 64 + i, n_in, n_out,
                                      mode=mode, d_lo=d_lo, d_hi=d_hi)
        L["attn_norm"] = rng.uniform(0.9, 1.1, cfg["n_embd"]).astype(np.float32)
        L["ffn_norm"] = rng.uniform(0.9, 1.1, cfg["n_embd"]).astype(np.float32)
        if biases:
            qd, kvd = shapes["attn_q"][1], shapes["attn_k"][1]
            L["bq"] = rng.uniform(-0.1, 0.1, qd).astype(np.float32)
            L["bk"] = rng.uniform(-0.1, 0.1, kvd).astype(np.float32)
            L["bv"] = rng.uniform(-0.1, 0.1, kvd).astype(np.float32)
        layers.append(L)
    emb = Weight.generate(ctx, mix["token_embd"], seed * 7 + 1, cfg["n_embd"], cfg["vocab"],
                          mode=mode, d_lo=d_lo, d_hi=d_hi)
    out = Weight.generate(ctx, mix["output"], seed * 7 + 2, cfg["n_embd"], cfg["vocab"],
                          mode=mode, d_lo=d_lo, d_hi=d_hi)
    onorm = rng.uniform(0.9, 1.1, cfg["n_embd"]).astype(np.float32)
    return ResidentForward(ctx, cfg, layers, emb, onorm, out)


# config 4: 27B-scale hybrid: 64 layers, full attention every 4th (24 q / 4 kv
# x 256, partial RoPE of 64 dims), 48 delta-net layers of 16 heads x 128
QWEN35_27B = dict(n_layer=64, n_embd=5120, n_head=24, n_head_kv=4, head_dim=256, n_ff=17408,
                  vocab=248320, rope_dim=64, ctx=4096, rms_eps=1e-6, freq_base=1e7,
                  full_attn_interval=4, dn_k_heads=16, dn_v_heads=16, dn_state=128, dn_conv=4)
HYBRID_MIX = dict(Q4_K_M_MIX, ssm_qkv=Q4_K, ssm_gate=Q4_K, ssm_out=Q4_K)


def hybrid_layer_shapes(cfg, l):
    """(n_in, n_out) of the quantized matrices of hybrid layer l."""
    E, ff = cfg["n_embd"], cfg["n_ff"]
    sh = dict(ffn_gate=(E, ff), ffn_up=(E, ff), ffn_down=(ff, E))
    if (l + 1) % cfg["full_attn_interval"] == 0:
        qd, kvd = cfg["n_head"] * cfg["head_dim"], cfg["n_head_kv"] * cfg["head_dim"]
        sh.update(attn_q=(E, 2 * qd), attn_k=(E, kvd), attn_v=(E, kvd), attn_output=(qd, E))
    else:
        vd = cfg["dn_v_heads"] * cfg["dn_state"]
        cd = (2 * cfg["dn_k_heads"] + cfg["dn_v_heads"]) * cfg["dn_state"]
        sh.update(ssm_qkv=(E, cd), ssm_gate=(E, vd), ssm_out=(vd, E))
    return sh


def synthetic_hybrid_model(ctx: Context, cfg: dict, seed: int = 1, mix: dict | None = None,
                           mode: int = 0, d_lo: float = 1e-3, d_hi: float = 1e-2):
    """Random-init hybrid model with weights generated on the GPU; f32 vectors
    drawn like the test models (norms ~U[0.9, 1.1], gate rows ~U[+-1.7/sqrt(E)],
    ssm_a ~U[-1, -0.1], dt ~U[-1, 1], conv taps ~U[-0.5, 0.5])."""
    mix = dict(HYBRID_MIX, **(mix or {}))
    rng = np.random.default_rng(seed)
    E = cfg["n_embd"]
    layers = []
    for l in range(cfg["n_layer"]):
        L = {}
        for i, (name, (n_in, n_out)) in enumerate(sorted(hybrid_layer_shapes(cfg, l).items())):
            L[name] = Weight.generate(ctx, mix[name], seed * 1000003 + l * 64 + i, n_in, n_out,
                                      mode=mode, d_lo=d_lo, d_hi=d_hi)
        L["attn_norm"] = rng.uniform(0.9, 1.1, E).astype(np.float32)
        L["post_norm"] = rng.uniform(0.9, 1.1, E).astype(np.float32)
        if (l + 1) % cfg["full_attn_interval"] == 0:
            L["q_norm"] = rng.uniform(0.9, 1.1, cfg["head_dim"]).astype(np.float32)
            L["k_norm"] = rng.uniform(0.9, 1.1, cfg["head_dim"]).astype(np.float32)
        else:
            nv, r = cfg["dn_v_heads"], 1.7 / np.sqrt(E)
            cd = (2 * cfg["dn_k_heads"] + nv) * cfg["dn_state"]
            L["ssm_alpha"] = rng.uniform(-r, r, nv * E).astype(np.float32)
            L["ssm_beta"] = rng.uniform(-r, r, nv * E).astype(np.float32)
            L["ssm_a"] = rng.uniform(-1.0, -0.1, nv).astype(np.float32)
            L["ssm_dt"] = rng.uniform(-1.0, 1.0, nv).astype(np.float32)
            L["ssm_conv"] = rng.uniform(-0.5, 0.5, cd * cfg["dn_conv"]).astype(np.float32)
            L["ssm_norm"] = rng.uniform(0.9, 1.1, cfg["dn_state"]).astype(np.float32)
        layers.append(L)
    emb = Weight.generate(ctx, mix["token_embd"], seed * 7 + 1, E, cfg["vocab"],
                          mode=mode, d_lo=d_lo, d_hi=d_hi)
    out = Weight.generate(ctx, mix["output"], seed * 7 + 2, E, cfg["vocab"],
                          mode=mode, d_lo=d_lo, d_hi=d_hi)
    onorm = rng.uniform(0.9, 1.1, E).astype(np.float32)
    return HybridForward(ctx, cfg, layers, emb, onorm, out)


__all__ = ["ResidentForward", "HybridForward", "synthetic_model", "synthetic_hybrid_model",
           "QWEN25_32B", "QWEN35_27B", "Q4_K_M_MIX", "HYBRID_MIX", "layer_shapes",
           "hybrid_layer_shapes", "ModelError"]
