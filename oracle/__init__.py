"""ctypes binding of the CPU oracle (``oracle/liblrs_oracle.so``).

TEST INFRASTRUCTURE ONLY: this module is the parity checker used by ``tests/``,
``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py``.  The
product package (``llama.rs_amd``) never imports it.

The C sources restate llama.rs's reference CPU path (``ggml-cpu`` dequant and
the ``llama-model`` f32 forward); each C function cites the reference
file:line it follows.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liblrs_oracle.so")

F32, F16, Q4_0, Q8_0, Q4_K, Q5_K, Q6_K = 0, 1, 2, 8, 12, 13, 14
BLOCK = {F32: 1, F16: 1, Q4_0: 32, Q8_0: 32, Q4_K: 256, Q5_K: 256, Q6_K: 256}
TYPE_SIZE = {F32: 4, F16: 2, Q4_0: 18, Q8_0: 34, Q4_K: 144, Q5_K: 176, Q6_K: 210}


def build(force: bool = False) -> str:
    """Compile the oracle with its Makefile (gcc, -ffp-contract=off)."""
    if force and os.path.exists(LIB_PATH):
        os.remove(LIB_PATH)
    subprocess.run(["make", "-s", "-C", HERE, "liblrs_oracle.so"], check=True)
    return LIB_PATH


def use_timing_build(out_dir: str) -> str:
    """Compile the same sources with ``-O3 -march=native`` (floating-point
    contraction allowed) into ``out_dir`` on the host that runs it, and make
    every later call of this module use that library.  It is the CPU
    baseline's timing build; the parity tests use the exact build above."""
    global LIB_PATH, _lib
    path = os.path.join(out_dir, "liblrs_oracle_timing.so")
    subprocess.run(["make", "-s", "-C", HERE, "timing", f"TIMING_OUT={path}"], check=True)
    LIB_PATH, _lib = path, None
    return path


_lib = None


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = C.CDLL(LIB_PATH)
        u8p, f32p, u32p = C.POINTER(C.c_uint8), C.POINTER(C.c_float), C.POINTER(C.c_uint32)
        L.lrso_block_size.restype = C.c_int64
        L.lrso_type_size.restype = C.c_int64
        L.lrso_f16_to_f32.restype = C.c_float
        L.lrso_f16_to_f32.argtypes = [C.c_uint16]
        L.lrso_f32_to_f16.restype = C.c_uint16
        L.lrso_f32_to_f16.argtypes = [C.c_float]
        L.lrso_dequant.restype = C.c_int64
        L.lrso_dequant.argtypes = [C.c_uint32, u8p, C.c_size_t, f32p]
        L.lrso_matvec.restype = C.c_int
        L.lrso_matvec.argtypes = [C.c_uint32, u8p, C.c_size_t, C.c_uint32, C.c_uint32,
                                  f32p, f32p, C.c_uint32, C.c_int]
        L.lrso_quantize_q8_0.restype = C.c_int
        L.lrso_quantize_q8_0.argtypes = [f32p, C.c_uint32, C.c_int, u8p]
        L.lrso_matvec_q8_0_actq.restype = C.c_int
        L.lrso_matvec_q8_0_actq.argtypes = [u8p, C.c_size_t, C.c_uint32, C.c_uint32, f32p,
                                            C.c_int, f32p]
        L.lrso_hash.restype = C.c_uint64
        L.lrso_hash.argtypes = [C.c_uint64, C.c_uint64, C.c_uint32]
        L.lrso_gen_blocks.restype = C.c_int
        L.lrso_gen_blocks.argtypes = [C.c_uint32, C.c_uint64, C.c_uint64, C.c_uint64, C.c_int,
                                      C.c_float, C.c_float, u8p]
        L.lrso_gen_uniform.argtypes = [C.c_uint64, C.c_uint64, C.c_float, C.c_float, f32p]
        L.lrso_gen_normal.argtypes = [C.c_uint64, C.c_uint64, f32p]
        L.lrso_rmsnorm_scale.argtypes = [f32p, f32p, C.c_uint32, C.c_uint32, C.c_float, f32p]
        L.lrso_freq_table.argtypes = [C.c_float, C.c_uint32, f32p]
        L.lrso_rope_norm.argtypes = [f32p, C.c_uint32, C.c_uint32, C.c_uint32, C.c_uint32,
                                     f32p, C.c_uint32]
        L.lrso_swiglu.argtypes = [f32p, f32p, C.c_uint32, f32p]
        L.lrso_softmax.argtypes = [f32p, C.c_uint32]
        L.lrso_argmax.restype = C.c_uint32
        L.lrso_argmax.argtypes = [f32p, C.c_uint32]
        L.lrso_attention.argtypes = [f32p, f32p, f32p, C.c_uint32, C.c_uint32, C.c_uint32,
                                     C.c_uint32, C.c_uint32, f32p]
        L.lrso_model_create.restype = C.c_void_p
        L.lrso_model_create.argtypes = [C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p,
                                        C.c_void_p, C.c_int, C.c_int]
        L.lrso_model_forward.restype = C.c_int
        L.lrso_model_forward.argtypes = [C.c_void_p, u32p, C.c_uint32, f32p]
        L.lrso_model_forward_partial.restype = C.c_int
        L.lrso_model_forward_partial.argtypes = [C.c_void_p, u32p, C.c_uint32, C.c_uint32]
        L.lrso_model_set_q8_actq.argtypes = [C.c_void_p, C.c_int]
        L.lrso_model_len.restype = C.c_uint32
        L.lrso_model_len.argtypes = [C.c_void_p]
        L.lrso_model_reset.argtypes = [C.c_void_p]
        L.lrso_model_destroy.argtypes = [C.c_void_p]
        L.lrso_softplus.restype = C.c_float
        L.lrso_softplus.argtypes = [C.c_float]
        L.lrso_sigmoid.restype = C.c_float
        L.lrso_sigmoid.argtypes = [C.c_float]
        L.lrso_silu.restype = C.c_float
        L.lrso_silu.argtypes = [C.c_float]
        L.lrso_l2_norm_rows.argtypes = [f32p, C.c_uint32, C.c_uint32, C.c_float]
        L.lrso_conv1d_step.argtypes = [f32p, f32p, f32p, C.c_uint32, C.c_uint32, f32p]
        L.lrso_delta_net_step.argtypes = [f32p, f32p, f32p, f32p, C.c_float, C.c_float,
                                          C.c_uint32, f32p]
        L.lrso_hybrid_create.restype = C.c_void_p
        L.lrso_hybrid_create.argtypes = [C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p,
                                         C.c_void_p, C.c_int, C.c_int]
        L.lrso_hybrid_forward.restype = C.c_int
        L.lrso_hybrid_forward.argtypes = [C.c_void_p, u32p, C.c_uint32, f32p]
        L.lrso_hybrid_len.restype = C.c_uint32
        L.lrso_hybrid_len.argtypes = [C.c_void_p]
        L.lrso_hybrid_reset.argtypes = [C.c_void_p]
        L.lrso_hybrid_destroy.argtypes = [C.c_void_p]
        _lib = L
    return _lib


def _u8(a: np.ndarray):
    return a.ctypes.data_as(C.POINTER(C.c_uint8))


def _f32(a: np.ndarray):
    return a.ctypes.data_as(C.POINTER(C.c_float))


def _u32(a: np.ndarray):
    return a.ctypes.data_as(C.POINTER(C.c_uint32))


def _as_u8(b) -> np.ndarray:
    if isinstance(b, (bytes, bytearray)):
        return np.frombuffer(bytes(b), dtype=np.uint8)
    return np.ascontiguousarray(b, dtype=np.uint8)


def row_bytes(t: int, n_in: int) -> int:
    return n_in // BLOCK[t] * TYPE_SIZE[t]


def f16_to_f32(h: int) -> float:
    return lib().lrso_f16_to_f32(int(h))


def f32_to_f16(f: float) -> int:
    return lib().lrso_f32_to_f16(float(f))


def dequant(t: int, data) -> np.ndarray:
    a = _as_u8(data)
    n = len(a) // TYPE_SIZE[t] * BLOCK[t] if len(a) % TYPE_SIZE[t] == 0 else 0
    out = np.zeros(max(n, 1), dtype=np.float32)
    rc = lib().lrso_dequant(t, _u8(a), len(a), _f32(out))
    if rc < 0:
        raise ValueError(f"dequant error {rc} (type {t}, {len(a)} bytes)")
    return out[:rc]


def matvec(t: int, w, n_in: int, n_out: int, x: np.ndarray, threads: int = 1) -> np.ndarray:
    a = _as_u8(w)
    x = np.ascontiguousarray(x, dtype=np.float32)
    cols = x.size // n_in
    y = np.zeros(cols * n_out, dtype=np.float32)
    rc = lib().lrso_matvec(t, _u8(a), len(a), n_in, n_out, _f32(x), _f32(y), cols, threads)
    if rc != 0:
        raise ValueError(f"matvec error {rc}")
    return y.reshape(cols, n_out) if x.ndim == 2 else y


def quantize_q8_0(x: np.ndarray, half_even: bool = True) -> np.ndarray:
    """GGUF Q8_0 bytes of x (ops.rs:284-368; half_even: the AVX2 rounding)."""
    x = np.ascontiguousarray(x, dtype=np.float32).ravel()
    out = np.zeros(x.size // 32 * 34, dtype=np.uint8)
    if lib().lrso_quantize_q8_0(_f32(x), x.size, int(half_even), _u8(out)) != 0:
        raise ValueError("n must be a multiple of 32")
    return out


def matvec_q8_0_actq(w, n_in: int, n_out: int, x: np.ndarray,
                     half_even: bool = True) -> np.ndarray:
    """matmul_q8_0_actq of one column (ops.rs:704-724, 728-886)."""
    a = _as_u8(w)
    x = np.ascontiguousarray(x, dtype=np.float32).ravel()
    y = np.zeros(n_out, dtype=np.float32)
    if lib().lrso_matvec_q8_0_actq(_u8(a), len(a), n_in, n_out, _f32(x), int(half_even),
                                   _f32(y)) != 0:
        raise ValueError("bad Q8_0 actq shape")
    return y


def gen_blocks(t: int, seed: int, n_blocks: int, block0: int = 0, mode: int = 0,
               d_lo: float = 1e-3, d_hi: float = 1e-2) -> np.ndarray:
    out = np.zeros(n_blocks * TYPE_SIZE[t], dtype=np.uint8)
    rc = lib().lrso_gen_blocks(t, seed, block0, n_blocks, mode, d_lo, d_hi, _u8(out))
    if rc != 0:
        raise ValueError(f"gen_blocks error {rc}")
    return out


def gen_weight(t: int, seed: int, n_out: int, n_in: int, **kw) -> np.ndarray:
    return gen_blocks(t, seed, n_out * (n_in // BLOCK[t]), **kw)


def gen_uniform(seed: int, n: int, lo: float, hi: float) -> np.ndarray:
    out = np.zeros(n, dtype=np.float32)
    lib().lrso_gen_uniform(seed, n, lo, hi, _f32(out))
    return out


def gen_normal(seed: int, n: int) -> np.ndarray:
    out = np.zeros(n, dtype=np.float32)
    lib().lrso_gen_normal(seed, n, _f32(out))
    return out


def rmsnorm_scale(x: np.ndarray, w: np.ndarray, eps: float) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    w = np.ascontiguousarray(w, dtype=np.float32)
    dim = w.size
    out = np.zeros_like(x)
    lib().lrso_rmsnorm_scale(_f32(x), _f32(w), x.size // dim, dim, eps, _f32(out))
    return out


def freq_table(base: float, rope_dim: int) -> np.ndarray:
    out = np.zeros(rope_dim // 2, dtype=np.float32)
    lib().lrso_freq_table(base, rope_dim, _f32(out))
    return out


def rope_norm(x: np.ndarray, n_tok: int, n_head: int, head_dim: int, rope_dim: int,
              freq: np.ndarray, pos0: int) -> np.ndarray:
    y = np.array(x, dtype=np.float32, copy=True)
    fr = np.ascontiguousarray(freq, dtype=np.float32)
    lib().lrso_rope_norm(_f32(y), n_tok, n_head, head_dim, rope_dim, _f32(fr), pos0)
    return y


def swiglu(g: np.ndarray, u: np.ndarray) -> np.ndarray:
    g = np.ascontiguousarray(g, dtype=np.float32)
    u = np.ascontiguousarray(u, dtype=np.float32)
    out = np.zeros_like(g)
    lib().lrso_swiglu(_f32(g), _f32(u), g.size, _f32(out))
    return out


def softmax(z: np.ndarray) -> np.ndarray:
    y = np.array(z, dtype=np.float32, copy=True)
    lib().lrso_softmax(_f32(y), y.size)
    return y


def argmax(v: np.ndarray) -> int:
    v = np.ascontiguousarray(v, dtype=np.float32)
    return int(lib().lrso_argmax(_f32(v), v.size))


def attention(q, k_cache, v_cache, n_tok, pos0, n_head, n_head_kv, head_dim) -> np.ndarray:
    q = np.ascontiguousarray(q, dtype=np.float32)
    k = np.ascontiguousarray(k_cache, dtype=np.float32)
    v = np.ascontiguousarray(v_cache, dtype=np.float32)
    out = np.zeros(n_tok * n_head * head_dim, dtype=np.float32)
    lib().lrso_attention(_f32(q), _f32(k), _f32(v), n_tok, pos0, n_head, n_head_kv,
                         head_dim, _f32(out))
    return out


def l2_norm_rows(x, dim, eps):
    y = np.array(x, dtype=np.float32, copy=True)
    lib().lrso_l2_norm_rows(_f32(y), y.size // dim, dim, eps)
    return y


def conv1d_step(state, x, w, d_conv):
    st = np.array(state, dtype=np.float32, copy=True)
    x = np.ascontiguousarray(x, dtype=np.float32)
    w = np.ascontiguousarray(w, dtype=np.float32)
    out = np.zeros_like(x)
    lib().lrso_conv1d_step(_f32(st), _f32(x), _f32(w), x.size, d_conv, _f32(out))
    return out, st


def delta_net_step(state, q, k, v, g, beta):
    st = np.array(state, dtype=np.float32, copy=True)
    q, k, v = (np.ascontiguousarray(a, dtype=np.float32) for a in (q, k, v))
    out = np.zeros_like(q)
    lib().lrso_delta_net_step(_f32(st), _f32(q), _f32(k), _f32(v), g, beta, q.size, _f32(out))
    return out, st


# ---------------------------------------------------------------------------
# dense model (model.rs:99-266)
# ---------------------------------------------------------------------------
class _Cfg(C.Structure):
    _fields_ = [(n, C.c_uint32) for n in
                ("n_layer", "n_embd", "n_head", "n_head_kv", "head_dim", "n_ff", "vocab",
                 "rope_dim", "ctx")] + [("rms_eps", C.c_float), ("freq_base", C.c_float)]


class _Tensor(C.Structure):
    _fields_ = [("type", C.c_uint32), ("bytes", C.c_void_p), ("len", C.c_size_t)]


class _Layer(C.Structure):
    _fields_ = [(n, _Tensor) for n in
                ("attn_norm", "attn_q", "attn_k", "attn_v", "attn_output", "ffn_norm",
                 "ffn_gate", "ffn_up", "ffn_down", "bq", "bk", "bv")]


LAYER_TENSORS = ("attn_norm", "attn_q", "attn_k", "attn_v", "attn_output", "ffn_norm",
                 "ffn_gate", "ffn_up", "ffn_down", "bq", "bk", "bv")


def _tensor(t):
    if t is None:
        return _Tensor(0, None, 0)
    ty, arr = t
    return _Tensor(ty, arr.ctypes.data, arr.nbytes)


class Model:
    """Oracle forward over a weight dict produced by ``tests/modelgen.py``.

    ``weights`` maps names to ``(type, np.ndarray[uint8 or float32])``; the
    arrays must outlive the model (they are borrowed)."""

    def __init__(self, cfg: dict, weights: dict, kv_f16: bool = True, threads: int = 1,
                 q8_actq: bool = True):
        self.cfg = cfg
        self._keep = weights
        c = _Cfg(cfg["n_layer"], cfg["n_embd"], cfg["n_head"], cfg["n_head_kv"],
                 cfg["head_dim"], cfg["n_ff"], cfg["vocab"], cfg["rope_dim"], cfg["ctx"],
                 cfg["rms_eps"], cfg["freq_base"])
        layers = (_Layer * cfg["n_layer"])()
        for i in range(cfg["n_layer"]):
            for n in LAYER_TENSORS:
                setattr(layers[i], n, _tensor(weights.get(f"blk.{i}.{n}")))
        self._c, self._layers = c, layers
        self._embd = _tensor(weights["token_embd"])
        self._onorm = _tensor(weights["output_norm"])
        self._out = _tensor(weights["output"])
        h = lib().lrso_model_create(C.byref(c), C.byref(self._embd), layers,
                                    C.byref(self._onorm), C.byref(self._out),
                                    1 if kv_f16 else 0, threads)
        if not h:
            raise ValueError("oracle model: bad shapes")
        self._h = h
        # Q8_0 weights: the reference forward's int8-activation path
        # (weights.rs:113-117), or dequant + f32 matmul when False
        lib().lrso_model_set_q8_actq(h, int(q8_actq))

    def forward(self, tokens) -> np.ndarray:
        toks = np.ascontiguousarray(tokens, dtype=np.uint32)
        logits = np.zeros(self.cfg["vocab"], dtype=np.float32)
        rc = lib().lrso_model_forward(self._h, _u32(toks), toks.size, _f32(logits))
        if rc != 0:
            raise ValueError(f"oracle forward error {rc}")
        return logits

    def forward_partial(self, tokens, n_layers: int) -> None:
        toks = np.ascontiguousarray(tokens, dtype=np.uint32)
        rc = lib().lrso_model_forward_partial(self._h, _u32(toks), toks.size, n_layers)
        if rc != 0:
            raise ValueError(f"oracle forward error {rc}")

    def __len__(self) -> int:
        return int(lib().lrso_model_len(self._h))

    def reset(self) -> None:
        lib().lrso_model_reset(self._h)

    def close(self) -> None:
        if self._h:
            lib().lrso_model_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


# ---------------------------------------------------------------------------
# hybrid attention + gated delta-net model (qwen35)
# ---------------------------------------------------------------------------
class _HybridCfg(C.Structure):
    _fields_ = [("base", _Cfg)] + [(n, C.c_uint32) for n in
                                   ("full_attn_interval", "dn_k_heads", "dn_v_heads",
                                    "dn_state", "dn_conv")]


HYBRID_TENSORS = ("attn_norm", "post_norm", "ffn_gate", "ffn_up", "ffn_down",
                  "attn_q", "attn_k", "attn_v", "attn_output", "q_norm", "k_norm",
                  "ssm_qkv", "ssm_gate", "ssm_out", "ssm_alpha", "ssm_beta", "ssm_a", "ssm_dt",
                  "ssm_conv", "ssm_norm")


class _HybridLayer(C.Structure):
    _fields_ = [(n, _Tensor) for n in HYBRID_TENSORS]


class HybridModel:
    """Oracle forward of the hybrid (full attention every
    ``full_attn_interval``-th layer, gated delta-net elsewhere) model over a
    weight dict produced by ``tests/modelgen.py``; arrays are borrowed."""

    def __init__(self, cfg: dict, weights: dict, kv_f16: bool = True, threads: int = 1):
        self.cfg = cfg
        self._keep = weights
        base = _Cfg(cfg["n_layer"], cfg["n_embd"], cfg["n_head"], cfg["n_head_kv"],
                    cfg["head_dim"], cfg["n_ff"], cfg["vocab"], cfg["rope_dim"], cfg["ctx"],
                    cfg["rms_eps"], cfg["freq_base"])
        c = _HybridCfg(base, cfg["full_attn_interval"], cfg["dn_k_heads"], cfg["dn_v_heads"],
                       cfg["dn_state"], cfg["dn_conv"])
        layers = (_HybridLayer * cfg["n_layer"])()
        for i in range(cfg["n_layer"]):
            for n in HYBRID_TENSORS:
                setattr(layers[i], n, _tensor(weights.get(f"blk.{i}.{n}")))
        self._c, self._layers = c, layers
        self._embd = _tensor(weights["token_embd"])
        self._onorm = _tensor(weights["output_norm"])
        self._out = _tensor(weights["output"])
        h = lib().lrso_hybrid_create(C.byref(c), C.byref(self._embd), layers,
                                     C.byref(self._onorm), C.byref(self._out),
                                     1 if kv_f16 else 0, threads)
        if not h:
            raise ValueError("oracle hybrid model: bad shapes")
        self._h = h

    def forward(self, tokens) -> np.ndarray:
        toks = np.ascontiguousarray(tokens, dtype=np.uint32)
        logits = np.zeros(self.cfg["vocab"], dtype=np.float32)
        rc = lib().lrso_hybrid_forward(self._h, _u32(toks), toks.size, _f32(logits))
        if rc != 0:
            raise ValueError(f"oracle hybrid forward error {rc}")
        return logits

    def __len__(self) -> int:
        return int(lib().lrso_hybrid_len(self._h))

    def reset(self) -> None:
        lib().lrso_hybrid_reset(self._h)

    def close(self) -> None:
        if self._h:
            lib().lrso_hybrid_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
