"""GGUF files: a v3 writer, the ctypes view of liblrs.so's reader, and the
model loader (lrs_model_load_gguf).

The reader mirrors gguf::GgufFile (crates/gguf/src/file.rs, parse.rs); the
writer produces what that parser reads (the layout of GgufBuilder,
crates/gguf/src/test_support.rs): header "GGUF", version 3, tensor count,
KV count, the KV pairs, the tensor infos, padding to general.alignment, the
tensor data.  write_synthetic writes random-init models of the configs'
shapes with weights generated on the GPU (seeded GGUF blocks) and read back
as GGUF bytes.
"""
from __future__ import annotations

import ctypes as C
import struct

import numpy as np

from . import Context, ModelError, Weight, check, lib, F32, Q4_K, Q6_K

_VT = {"u8": 0, "i8": 1, "u16": 2, "i16": 3, "u32": 4, "i32": 5, "f32": 6, "bool": 7, "str": 8,
       "arr": 9, "u64": 10, "i64": 11, "f64": 12}
_FMT = {0: "<B", 1: "<b", 2: "<H", 3: "<h", 4: "<I", 5: "<i", 6: "<f", 7: "<B", 10: "<Q",
        11: "<q", 12: "<d"}
BLOCK = {0: (1, 4), 1: (1, 2), 2: (32, 18), 8: (32, 34), 12: (256, 144), 13: (256, 176),
         14: (256, 210)}


def _bind():
    vp, u32p, u64p, sz = C.c_void_p, C.POINTER(C.c_uint32), C.POINTER(C.c_uint64), C.c_size_t
    sig = {
        "lrs_gguf_open": (C.c_int, [C.c_char_p, C.POINTER(vp)]),
        "lrs_gguf_close": (None, [vp]),
        "lrs_gguf_version": (C.c_uint32, [vp]),
        "lrs_gguf_n_tensors": (C.c_uint64, [vp]),
        "lrs_gguf_get_u32": (C.c_int, [vp, C.c_char_p, u32p]),
        "lrs_gguf_get_f32": (C.c_int, [vp, C.c_char_p, C.POINTER(C.c_float)]),
        "lrs_gguf_get_str": (C.c_int, [vp, C.c_char_p, C.POINTER(C.c_char_p)]),
        "lrs_gguf_array_len": (C.c_int, [vp, C.c_char_p, u64p]),
        "lrs_gguf_tensor": (C.c_int, [vp, C.c_char_p, u32p, u64p, u32p, C.POINTER(vp),
                                      C.POINTER(sz)]),
        "lrs_model_load_gguf": (C.c_int, [vp, vp, C.c_uint32, C.POINTER(vp)]),
    }
    for name, (res, args) in sig.items():
        f = getattr(lib, name)
        f.restype = res
        f.argtypes = args


_bind()


# ---------------------------------------------------------------------------
# writer
# ---------------------------------------------------------------------------
def _str(s: str) -> bytes:
    b = s.encode()
    return struct.pack("<Q", len(b)) + b


def _value(kind: str, v) -> bytes:
    t = _VT[kind]
    if kind == "str":
        return struct.pack("<I", t) + _str(v)
    if kind == "arr":
        et, items = v  # (element kind, list)
        out = struct.pack("<IIQ", t, _VT[et], len(items))
        if et == "str":
            return out + b"".join(_str(x) for x in items)
        return out + b"".join(struct.pack(_FMT[_VT[et]], x) for x in items)
    return struct.pack("<I", t) + struct.pack(_FMT[t], v)


def write_gguf(path: str, kv: list, tensors: list, alignment: int = 32) -> None:
    """kv: [(key, kind, value)], kind in u8..f64 / "str" / "arr" (value =
    (element kind, items)); tensors: [(name, ggml type, dims, bytes)] with
    dims[0] the row length.  Tensor data offsets are aligned to `alignment`."""
    kvs = list(kv)
    if alignment != 32 and not any(k == "general.alignment" for k, _, _ in kvs):
        kvs.append(("general.alignment", "u32", alignment))
    head = b"GGUF" + struct.pack("<IQQ", 3, len(tensors), len(kvs))
    head += b"".join(_str(k) + _value(kind, v) for k, kind, v in kvs)
    infos, blobs, off = b"", [], 0
    for name, t, dims, data in tensors:
        data = bytes(data)
        be, bb = BLOCK[t]
        n = int(np.prod(dims))
        if n % be or len(data) != n // be * bb:
            raise ValueError(f"{name}: {len(data)} bytes for dims {dims} of type {t}")
        infos += _str(name) + struct.pack("<I", len(dims)) + \
            b"".join(struct.pack("<Q", d) for d in dims) + struct.pack("<IQ", t, off)
        pad = (-len(data)) % alignment
        blobs.append(data + b"\0" * pad)
        off += len(data) + pad
    meta = head + infos
    meta += b"\0" * ((-len(meta)) % alignment)
    with open(path, "wb") as f:
        f.write(meta)
        for b in blobs:
            f.write(b)


# ---------------------------------------------------------------------------
# reader (liblrs.so)
# ---------------------------------------------------------------------------
class GgufFile:
    """A mapped GGUF file (lrs_gguf_open); tensor() returns the raw bytes."""

    def __init__(self, path: str):
        h = C.c_void_p()
        check(lib.lrs_gguf_open(path.encode(), C.byref(h)))
        self.h = h

    @property
    def version(self) -> int:
        return int(lib.lrs_gguf_version(self.h))

    @property
    def n_tensors(self) -> int:
        return int(lib.lrs_gguf_n_tensors(self.h))

    def u32(self, key: str) -> int:
        v = C.c_uint32()
        check(lib.lrs_gguf_get_u32(self.h, key.encode(), C.byref(v)))
        return int(v.value)

    def f32(self, key: str) -> float:
        v = C.c_float()
        check(lib.lrs_gguf_get_f32(self.h, key.encode(), C.byref(v)))
        return float(v.value)

    def str(self, key: str) -> str:
        v = C.c_char_p()
        check(lib.lrs_gguf_get_str(self.h, key.encode(), C.byref(v)))
        return v.value.decode()

    def array_len(self, key: str) -> int:
        v = C.c_uint64()
        check(lib.lrs_gguf_array_len(self.h, key.encode(), C.byref(v)))
        return int(v.value)

    def tensor(self, name: str):
        """(ggml type, dims, uint8 array copy of the bytes)"""
        t, nd = C.c_uint32(), C.c_uint32()
        dims = (C.c_uint64 * 4)()
        p, n = C.c_void_p(), C.c_size_t()
        check(lib.lrs_gguf_tensor(self.h, name.encode(), C.byref(t), dims, C.byref(nd),
                                  C.byref(p), C.byref(n)))
        data = np.frombuffer((C.c_uint8 * n.value).from_address(p.value), np.uint8).copy()
        return int(t.value), [int(dims[i]) for i in range(nd.value)], data

    def close(self) -> None:
        if getattr(self, "h", None):
            lib.lrs_gguf_close(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def load_gguf(ctx: Context, path: str, ctx_len: int = 0):
    """ResidentForward / HybridForward over a GGUF file (lrs_model_load_gguf)."""
    from .model import ResidentForward

    g = GgufFile(path)
    try:
        h = C.c_void_p()
        check(lib.lrs_model_load_gguf(ctx.h, g.h, ctx_len, C.byref(h)))
        arch = "llama"
        try:
            arch = g.str("general.architecture")
        except ModelError:
            pass
        vocab = g.array_len("tokenizer.ggml.tokens")
    finally:
        g.close()
    m = ResidentForward.__new__(ResidentForward)
    m.ctx, m.h, m.vocab, m._keep = ctx, h, vocab, []
    m.cfg = {"architecture": arch, "vocab": vocab}
    ctx._models.add(m)
    return m


# ---------------------------------------------------------------------------
# model -> GGUF (names of gpu.rs:128-600)
# ---------------------------------------------------------------------------
def model_kv(cfg: dict, arch: str) -> list:
    """The metadata LlamaConfig::from_gguf reads (config.rs:81-187)."""
    p = arch + "."
    kv = [("general.architecture", "str", arch),
          (p + "block_count", "u32", cfg["n_layer"]),
          (p + "embedding_length", "u32", cfg["n_embd"]),
          (p + "feed_forward_length", "u32", cfg["n_ff"]),
          (p + "attention.head_count", "u32", cfg["n_head"]),
          (p + "attention.head_count_kv", "u32", cfg["n_head_kv"]),
          (p + "attention.key_length", "u32", cfg["head_dim"]),
          (p + "rope.dimension_count", "u32", cfg["rope_dim"]),
          (p + "rope.freq_base", "f32", cfg["freq_base"]),
          (p + "attention.layer_norm_rms_epsilon", "f32", cfg["rms_eps"]),
          (p + "context_length", "u32", cfg["ctx"]),
          ("tokenizer.ggml.tokens", "arr", ("str", [f"t{i}" for i in range(cfg["vocab"])])),
          ("tokenizer.ggml.bos_token_id", "u32", 1),
          ("tokenizer.ggml.eos_token_id", "u32", 2)]
    if "full_attn_interval" in cfg:
        kv += [(p + "full_attention_interval", "u32", cfg["full_attn_interval"]),
               (p + "ssm.conv_kernel", "u32", cfg["dn_conv"]),
               (p + "ssm.inner_size", "u32", cfg["dn_v_heads"] * cfg["dn_state"]),
               (p + "ssm.state_size", "u32", cfg["dn_state"]),
               (p + "ssm.time_step_rank", "u32", cfg["dn_v_heads"]),
               (p + "ssm.group_count", "u32", cfg["dn_k_heads"])]
    return kv


# our layer-dict names -> GGUF tensor names
GGUF_NAMES = {"attn_q": "attn_q.weight", "attn_k": "attn_k.weight", "attn_v": "attn_v.weight",
              "attn_output": "attn_output.weight", "ffn_gate": "ffn_gate.weight",
              "ffn_up": "ffn_up.weight", "ffn_down": "ffn_down.weight",
              "attn_norm": "attn_norm.weight", "ffn_norm": "ffn_norm.weight",
              "post_norm": "post_attention_norm.weight", "bq": "attn_q.bias",
              "bk": "attn_k.bias", "bv": "attn_v.bias", "q_norm": "attn_q_norm.weight",
              "k_norm": "attn_k_norm.weight", "ssm_qkv": "attn_qkv.weight",
              "ssm_gate": "attn_gate.weight", "ssm_out": "ssm_out.weight",
              "ssm_alpha": "ssm_alpha.weight", "ssm_beta": "ssm_beta.weight", "ssm_a": "ssm_a",
              "ssm_dt": "ssm_dt.bias", "ssm_conv": "ssm_conv1d.weight",
              "ssm_norm": "ssm_norm.weight"}


def vector_dims(cfg: dict, name: str, n: int) -> list:
    if name in ("ssm_alpha", "ssm_beta"):
        return [cfg["n_embd"], cfg["dn_v_heads"]]
    if name == "ssm_conv":
        return [cfg["dn_conv"], n // cfg["dn_conv"]]
    return [n]


def write_synthetic(ctx: Context, path: str, cfg: dict, seed: int = 1, mix: dict | None = None,
                    mode: int = 0, d_lo: float = 1e-3, d_hi: float = 1e-2) -> None:
    """Random-init model of the given shape (dense, or hybrid when cfg has
    full_attn_interval) written as GGUF: weights generated on the GPU,
    downloaded as GGUF blocks, f32 vectors drawn as in model.py."""
    from .model import (HYBRID_MIX, Q4_K_M_MIX, hybrid_layer_shapes, layer_shapes)

    hybrid = "full_attn_interval" in cfg
    mix = dict(HYBRID_MIX if hybrid else Q4_K_M_MIX, **(mix or {}))
    rng = np.random.default_rng(seed)
    E = cfg["n_embd"]
    tensors = []

    def mat(name, t, n_in, n_out, s):
        w = Weight.generate(ctx, t, s, n_in, n_out, mode=mode, d_lo=d_lo, d_hi=d_hi)
        data = w.download()
        w.free()
        return (name, t, [n_in, n_out], data.tobytes())

    for l in range(cfg["n_layer"]):
        shapes = hybrid_layer_shapes(cfg, l) if hybrid else layer_shapes(cfg)
        for i, (name, (n_in, n_out)) in enumerate(sorted(shapes.items())):
            tensors.append(mat(f"blk.{l}.{GGUF_NAMES[name]}", mix[name], n_in, n_out,
                               seed * 1000003 + l * 64 + i))
        vecs = {"attn_norm": rng.uniform(0.9, 1.1, E)}
        if hybrid:
            vecs["post_norm"] = rng.uniform(0.9, 1.1, E)
            if (l + 1) % cfg["full_attn_interval"] == 0:
                vecs["q_norm"] = rng.uniform(0.9, 1.1, cfg["head_dim"])
                vecs["k_norm"] = rng.uniform(0.9, 1.1, cfg["head_dim"])
            else:
                nv, r = cfg["dn_v_heads"], 1.7 / np.sqrt(E)
                cd = (2 * cfg["dn_k_heads"] + nv) * cfg["dn_state"]
                vecs.update(ssm_alpha=rng.uniform(-r, r, nv * E), ssm_beta=rng.uniform(-r, r, nv * E),
                            ssm_a=rng.uniform(-1.0, -0.1, nv), ssm_dt=rng.uniform(-1.0, 1.0, nv),
                            ssm_conv=rng.uniform(-0.5, 0.5, cd * cfg["dn_conv"]),
                            ssm_norm=rng.uniform(0.9, 1.1, cfg["dn_state"]))
        else:
            vecs["ffn_norm"] = rng.uniform(0.9, 1.1, E)
        for name, a in vecs.items():
            a = np.ascontiguousarray(a, np.float32)
            tensors.append((f"blk.{l}.{GGUF_NAMES[name]}", F32, vector_dims(cfg, name, a.size),
                            a.tobytes()))
    tensors.append(mat("token_embd.weight", mix["token_embd"], E, cfg["vocab"], seed * 7 + 1))
    tensors.append(mat("output.weight", mix["output"], E, cfg["vocab"], seed * 7 + 2))
    tensors.append(("output_norm.weight", F32, [E],
                    rng.uniform(0.9, 1.1, E).astype(np.float32).tobytes()))
    write_gguf(path, model_kv(cfg, "qwen35" if hybrid else "qwen2"), tensors)


__all__ = ["write_gguf", "GgufFile", "load_gguf", "model_kv", "write_synthetic", "GGUF_NAMES",
           "vector_dims"]
