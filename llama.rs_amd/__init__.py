"""llama.rs_amd — MI355X (gfx950) batch-1 decode hot path of llama.rs.

Host-side mirror of the reference's GPU backend interface, over the C ABI of
``liblrs.so`` (``include/lrs.h``):

* :class:`GpuMatmul`     — ``llama_model::GpuMatmul`` (crates/llama-model/src/gpu.rs:1057-1065)
* :func:`dequant_to_f32` — ``ggml_cpu::dequant_to_f32`` (crates/ggml-cpu/src/dequant.rs:10-21)
* :class:`ResidentForward` (in :mod:`.model`) — ``llama_model::GpuResidentDecode``
  (gpu.rs:379-455) as implemented by ``llama_vulkan::ResidentForward``.

Errors from the library raise :class:`ModelError` carrying the library's
message, like ``ModelError::Gpu(String)`` (crates/llama-model/src/error.rs:26-27).
There is no CPU fallback: when ``liblrs.so`` is missing the import fails.
"""
from __future__ import annotations

import ctypes as C
import os
import weakref

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liblrs.so")

# GGUF type ids (crates/gguf/src/types.rs:84-107)
F32, F16, Q4_0, Q8_0, Q4_K, Q5_K, Q6_K = 0, 1, 2, 8, 12, 13, 14
BLOCK = {F32: 1, F16: 1, Q4_0: 32, Q8_0: 32, Q4_K: 256, Q5_K: 256, Q6_K: 256}
TYPE_SIZE = {F32: 4, F16: 2, Q4_0: 18, Q8_0: 34, Q4_K: 144, Q5_K: 176, Q6_K: 210}
TYPE_NAME = {F32: "F32", F16: "F16", Q4_0: "Q4_0", Q8_0: "Q8_0", Q4_K: "Q4_K", Q5_K: "Q5_K",
             Q6_K: "Q6_K"}


# largest n_in of lrs_matvec_dev_noalloc (LRS_NOALLOC_MAX_N_IN)
NOALLOC_MAX_N_IN = 46592


class ModelError(RuntimeError):
    """Mirror of llama_model::ModelError::Gpu(String)."""

    def __init__(self, code: int, msg: str):
        super().__init__(f"[{code}] {msg}")
        self.code = code


def _load() -> C.CDLL:
    if not os.path.exists(LIB_PATH):
        raise ImportError(f"{LIB_PATH} is not built; run __graft_entry__.build() "
                          "(python llama.rs_amd/build.py)")
    L = C.CDLL(LIB_PATH)
    vp, sz, u32, i32 = C.c_void_p, C.c_size_t, C.c_uint32, C.c_int
    pvp = C.POINTER(C.c_void_p)
    sig = {
        "lrs_last_error": (C.c_char_p, []),
        "lrs_version": (C.c_char_p, []),
        "lrs_ctx_create": (i32, [i32, pvp]),
        "lrs_ctx_destroy": (None, [vp]),
        "lrs_ctx_sync": (i32, [vp]),
        "lrs_ctx_mem_info": (i32, [vp, C.POINTER(sz), C.POINTER(sz)]),
        "lrs_weight_upload": (i32, [vp, u32, vp, sz, u32, u32, pvp]),
        "lrs_weight_generate": (i32, [vp, u32, C.c_uint64, i32, C.c_float, C.c_float, u32, u32,
                                      pvp]),
        "lrs_weight_download": (i32, [vp, vp, vp, sz]),
        "lrs_weight_gguf_bytes": (sz, [vp]),
        "lrs_weight_free": (None, [vp]),
        "lrs_dequant_f32": (i32, [vp, u32, vp, sz, vp]),
        "lrs_weight_dequant_dev": (i32, [vp, vp, vp]),
        "lrs_matvec_f32": (i32, [vp, vp, vp, vp, u32]),
        "lrs_matvec_dev": (i32, [vp, vp, vp, vp, u32]),
        "lrs_matvec_dev_noalloc": (i32, [vp, vp, vp, vp, u32]),
        "lrs_gemm_dev": (i32, [vp, vp, vp, vp, u32, i32]),
        "lrs_gemm_group_dev": (i32, [vp, vp, u32, vp, vp, u32, i32]),
        "lrs_quantize_q8_0_dev": (i32, [vp, vp, u32, i32, vp]),
        "lrs_matvec_q8_0_actq_dev": (i32, [vp, vp, vp, vp, u32, i32]),
        "lrs_dev_alloc": (i32, [vp, sz, pvp]),
        "lrs_dev_free": (i32, [vp, vp]),
        "lrs_copy_h2d": (i32, [vp, vp, vp, sz]),
        "lrs_copy_d2h": (i32, [vp, vp, vp, sz]),
        "lrs_matvec_set_geom": (i32, [i32, i32, i32]),
        "lrs_capture_begin": (i32, [vp]),
        "lrs_capture_end": (i32, [vp, pvp]),
        "lrs_graph_launch": (i32, [vp]),
        "lrs_graph_destroy": (None, [vp]),
        "lrs_timer_start": (i32, [vp]),
        "lrs_timer_stop": (i32, [vp, C.POINTER(C.c_float)]),
    }
    for name, (res, args) in sig.items():
        f = getattr(L, name)
        f.restype = res
        f.argtypes = args
    return L


lib = _load()


def check(rc: int) -> None:
    if rc != 0:
        raise ModelError(rc, lib.lrs_last_error().decode())


def _ptr(a: np.ndarray) -> int:
    return a.ctypes.data


def row_bytes(t: int, n_in: int) -> int:
    return n_in // BLOCK[t] * TYPE_SIZE[t]


class Graph:
    """A captured sequence of device work (lrs_capture_end); launch() replays
    it on the context stream."""

    def __init__(self, ctx, h):
        self.ctx, self.h = ctx, h

    def launch(self) -> None:
        check(lib.lrs_graph_launch(self.h))

    def close(self) -> None:
        if getattr(self, "h", None):
            lib.lrs_graph_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class Context:
    """A device + stream (VulkanContext/VulkanDevice in the reference)."""

    def __init__(self, device: int = 0):
        """Opens `device` (default 0: this process touches no other GPU);
        device = -1 asks lrs_ctx_create to pick the device with the most free
        HBM, which opens every visible device to compare them."""
        h = C.c_void_p()
        check(lib.lrs_ctx_create(device, C.byref(h)))
        self.h = h
        self.device = device if device >= 0 else None
        # children must be released before the context (C-ABI contract):
        # models first (they reference weights), then weights and buffers
        self._models = weakref.WeakSet()
        self._weights = weakref.WeakSet()
        self._bufs = weakref.WeakSet()

    def sync(self) -> None:
        check(lib.lrs_ctx_sync(self.h))

    def mem_info(self):
        f, t = C.c_size_t(), C.c_size_t()
        check(lib.lrs_ctx_mem_info(self.h, C.byref(f), C.byref(t)))
        return f.value, t.value

    def alloc(self, nbytes: int) -> "DeviceBuffer":
        return DeviceBuffer(self, nbytes)

    def timer_start(self) -> None:
        check(lib.lrs_timer_start(self.h))

    def capture(self, fn) -> "Graph":
        """Records the device work fn() enqueues on this context's stream
        (asynchronous *_dev calls only) into a replayable HIP graph."""
        check(lib.lrs_capture_begin(self.h))
        try:
            fn()
        finally:
            g = C.c_void_p()
            rc = lib.lrs_capture_end(self.h, C.byref(g))
        check(rc)
        graph = Graph(self, g)
        self._models.add(graph)
        return graph

    def timer_stop(self) -> float:
        ms = C.c_float()
        check(lib.lrs_timer_stop(self.h, C.byref(ms)))
        return ms.value

    def close(self) -> None:
        if getattr(self, "h", None):
            for group in (self._models, self._weights, self._bufs):
                for child in list(group):
                    child.close() if hasattr(child, "close") else child.free()
            lib.lrs_ctx_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def __enter__(self):
        return self

    def __exit__(self, *a):
        self.close()


class DeviceBuffer:
    def __init__(self, ctx: Context, nbytes: int):
        self.ctx, self.nbytes = ctx, nbytes
        p = C.c_void_p()
        check(lib.lrs_dev_alloc(ctx.h, nbytes, C.byref(p)))
        self.ptr = p.value
        ctx._bufs.add(self)

    def upload(self, a: np.ndarray) -> None:
        a = np.ascontiguousarray(a)
        assert a.nbytes <= self.nbytes
        check(lib.lrs_copy_h2d(self.ctx.h, self.ptr, _ptr(a), a.nbytes))

    def download(self, dtype, count: int) -> np.ndarray:
        out = np.empty(count, dtype=dtype)
        assert out.nbytes <= self.nbytes
        check(lib.lrs_copy_d2h(self.ctx.h, _ptr(out), self.ptr, out.nbytes))
        return out

    def free(self) -> None:
        if self.ptr and self.ctx.h:
            check(lib.lrs_dev_free(self.ctx.h, self.ptr))
        self.ptr = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class Weight:
    """A resident n_out x n_in GGUF tensor (QTensor uploaded by Uploader::tensor)."""

    def __init__(self, ctx: Context, handle, t: int, n_in: int, n_out: int):
        self.ctx, self.h, self.type, self.n_in, self.n_out = ctx, handle, t, n_in, n_out
        ctx._weights.add(self)

    @classmethod
    def upload(cls, ctx: Context, t: int, data, n_in: int, n_out: int) -> "Weight":
        a = np.ascontiguousarray(np.frombuffer(bytes(data), np.uint8)
                                 if isinstance(data, (bytes, bytearray)) else data)
        h = C.c_void_p()
        check(lib.lrs_weight_upload(ctx.h, t, _ptr(a), a.nbytes, n_in, n_out, C.byref(h)))
        return cls(ctx, h, t, n_in, n_out)

    @classmethod
    def generate(cls, ctx: Context, t: int, seed: int, n_in: int, n_out: int, mode: int = 0,
                 d_lo: float = 1e-3, d_hi: float = 1e-2) -> "Weight":
        h = C.c_void_p()
        check(lib.lrs_weight_generate(ctx.h, t, seed, mode, d_lo, d_hi, n_in, n_out,
                                      C.byref(h)))
        return cls(ctx, h, t, n_in, n_out)

    @property
    def gguf_bytes(self) -> int:
        return int(lib.lrs_weight_gguf_bytes(self.h))

    def download(self) -> np.ndarray:
        out = np.empty(self.gguf_bytes, np.uint8)
        check(lib.lrs_weight_download(self.ctx.h, self.h, _ptr(out), out.nbytes))
        return out

    def dequant_dev(self, out: DeviceBuffer) -> None:
        check(lib.lrs_weight_dequant_dev(self.ctx.h, self.h, out.ptr))

    def matvec(self, x: np.ndarray) -> np.ndarray:
        x = np.ascontiguousarray(x, dtype=np.float32)
        cols = x.size // self.n_in
        if cols * self.n_in != x.size:
            raise ModelError(-1, f"x has {x.size} elements, not a multiple of n_in={self.n_in}")
        y = np.empty(cols * self.n_out, np.float32)
        check(lib.lrs_matvec_f32(self.ctx.h, self.h, _ptr(x), _ptr(y), cols))
        return y.reshape(cols, self.n_out) if x.ndim == 2 else y

    def matvec_dev(self, x: DeviceBuffer, y: DeviceBuffer, cols: int = 1) -> None:
        check(lib.lrs_matvec_dev(self.ctx.h, self.h, x.ptr, y.ptr, cols))

    def matvec_dev_noalloc(self, x: DeviceBuffer, y: DeviceBuffer, cols: int = 1) -> None:
        """matvec_dev with the input pack in the library's static device array
        (no allocation; n_in <= NOALLOC_MAX_N_IN)."""
        check(lib.lrs_matvec_dev_noalloc(self.ctx.h, self.h, x.ptr, y.ptr, cols))

    def matvec_actq_dev(self, x: DeviceBuffer, y: DeviceBuffer, cols: int = 1,
                        half_even: bool = True) -> None:
        """matmul_q8_0_actq (ops.rs:728-886): x rounded to Q8_0 first (async)."""
        check(lib.lrs_matvec_q8_0_actq_dev(self.ctx.h, self.h, x.ptr, y.ptr, cols,
                                           int(half_even)))

    def matvec_actq(self, x: np.ndarray, half_even: bool = True) -> np.ndarray:
        """Host wrapper of matvec_actq_dev: x [cols, n_in] -> [cols, n_out]."""
        x = np.ascontiguousarray(x, dtype=np.float32)
        cols = x.size // self.n_in
        if cols * self.n_in != x.size:
            raise ModelError(-1, f"x has {x.size} elements, not a multiple of n_in={self.n_in}")
        xb, yb = self.ctx.alloc(x.nbytes), self.ctx.alloc(4 * cols * self.n_out)
        try:
            xb.upload(x)
            self.matvec_actq_dev(xb, yb, cols, half_even)
            self.ctx.sync()
            y = yb.download(np.float32, cols * self.n_out)
        finally:
            xb.free()
            yb.free()
        return y.reshape(cols, self.n_out) if x.ndim == 2 else y

    def gemm_dev(self, a: DeviceBuffer, y: DeviceBuffer, m: int, precision: int = 1) -> None:
        """Y[m][n_out] = A[m][n_in] W^T on the matrix cores (async, device buffers)."""
        check(lib.lrs_gemm_dev(self.ctx.h, self.h, a.ptr, y.ptr, m, precision))

    def gemm(self, a: np.ndarray, precision: int = 1) -> np.ndarray:
        """Host wrapper of gemm_dev: a [m, n_in] f32 -> [m, n_out] f32."""
        a = np.ascontiguousarray(a, dtype=np.float32)
        m = a.shape[0]
        ab, yb = self.ctx.alloc(a.nbytes), self.ctx.alloc(4 * m * self.n_out)
        try:
            ab.upload(a)
            self.gemm_dev(ab, yb, m, precision)
            self.ctx.sync()
            return yb.download(np.float32, m * self.n_out).reshape(m, self.n_out)
        finally:
            ab.free()
            yb.free()

    def free(self) -> None:
        if getattr(self, "h", None) and self.ctx.h:
            lib.lrs_weight_free(self.h)
        self.h = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


def dequant_to_f32(ctx: Context, t: int, data) -> np.ndarray:
    """ggml_cpu::dequant_to_f32 on the GPU, bit-exact (dequant.rs:10-21)."""
    a = np.ascontiguousarray(np.frombuffer(bytes(data), np.uint8)
                             if isinstance(data, (bytes, bytearray)) else data)
    if t not in TYPE_SIZE:
        raise ModelError(-5, f"unsupported type {t}")
    n = a.nbytes // TYPE_SIZE[t] * BLOCK[t]
    out = np.empty(max(n, 1), np.float32)
    check(lib.lrs_dequant_f32(ctx.h, t, _ptr(a), a.nbytes, _ptr(out)))
    return out[:n]


def quantize_q8_0(ctx: Context, x: np.ndarray, half_even: bool = True) -> np.ndarray:
    """quantize_q8_0 / quantize_q8_0_avx2 (ops.rs:284-368) on the GPU: GGUF
    Q8_0 bytes of x, bit-exact; half_even selects the AVX2 path's rounding."""
    x = np.ascontiguousarray(x, dtype=np.float32).ravel()
    if x.size == 0 or x.size % 32:
        raise ModelError(-1, "n must be a positive multiple of 32")
    nb = x.size // 32 * 34
    xb, qb = ctx.alloc(x.nbytes), ctx.alloc(nb)
    try:
        xb.upload(x)
        check(lib.lrs_quantize_q8_0_dev(ctx.h, xb.ptr, x.size, int(half_even), qb.ptr))
        ctx.sync()
        return qb.download(np.uint8, nb)
    finally:
        xb.free()
        qb.free()


def gemm_group(ctx: Context, weights, a: np.ndarray, precision: int = 1) -> list:
    """lrs_gemm_group_dev: the GEMM of each weight over the same a [m, n_in]
    as one launch; returns [m, n_out] f32 per weight."""
    a = np.ascontiguousarray(a, dtype=np.float32)
    m = a.shape[0]
    ab = ctx.alloc(a.nbytes)
    ys = [ctx.alloc(4 * m * w.n_out) for w in weights]
    try:
        ab.upload(a)
        wa = (C.c_void_p * len(weights))(*[w.h for w in weights])
        ya = (C.c_void_p * len(weights))(*[y.ptr for y in ys])
        check(lib.lrs_gemm_group_dev(ctx.h, wa, len(weights), ab.ptr, ya, m, precision))
        ctx.sync()
        return [y.download(np.float32, m * w.n_out).reshape(m, w.n_out) for y, w in zip(ys, weights)]
    finally:
        ab.free()
        for y in ys:
            y.free()


class GpuMatmul:
    """llama_model::GpuMatmul (gpu.rs:1057-1065): one matvec per call, weights
    uploaded on first use and cached by the buffer's identity, like the
    reference's ResidentGpu (crates/llama-vulkan/src/resident.rs:141-452)."""

    def __init__(self, ctx: Context | None = None):
        self.ctx = ctx or Context(0)
        self._cache: dict = {}

    def _weight(self, t, w_bytes, n_in, n_out) -> Weight:
        key = (t, id(w_bytes), n_in, n_out)
        w = self._cache.get(key)
        if w is None:
            w = Weight.upload(self.ctx, t, w_bytes, n_in, n_out)
            self._cache[key] = w
        return w

    def matvec_q8_0(self, w_bytes, x, n_in: int, n_out: int) -> np.ndarray:
        return self.matvec(Q8_0, w_bytes, x, n_in, n_out)

    def matvec(self, t: int, w_bytes, x, n_in: int, n_out: int) -> np.ndarray:
        return self._weight(t, w_bytes, n_in, n_out).matvec(np.asarray(x, np.float32))


# launch shapes of the plain matvec (tiles per wavefront, tile groups and
# K-slices per workgroup) that the library instantiates
MATVEC_GEOMS = [(1, 1, 4), (1, 2, 4), (1, 2, 2), (2, 4, 2), (2, 2, 4), (1, 2, 6)]


def set_matvec_geom(tiles_per_wave: int = 0, tile_groups: int = 0, k_slices: int = 0) -> None:
    """Tuning knob (LLAMA_RS_MATVEC_GEOM, resident_forward.rs:164-176); 0s = automatic."""
    check(lib.lrs_matvec_set_geom(tiles_per_wave, tile_groups, k_slices))


def version() -> str:
    return lib.lrs_version().decode()

