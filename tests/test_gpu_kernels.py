"""GPU parity of the kernel-level C ABI against the CPU oracle.

Bars: dequant bit-exact; matvec within 1e-4 relative
L2 of dequant + sequential f32 dot (measured values are ~1e-7).
"""
import json
import os

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

HERE = os.path.dirname(os.path.abspath(__file__))
F32, F16, Q4_0, Q8_0, Q4_K, Q5_K, Q6_K = 0, 1, 2, 8, 12, 13, 14
KQ = [Q8_0, Q4_K, Q5_K, Q6_K]
THREADS = min(16, os.cpu_count() or 1)
MATVEC_TOL = 1e-4


@pytest.fixture(scope="module")
def ctx(lrs):
    c = lrs.Context(0)
    yield c
    c.close()


def rel_l2(a, b):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))


def f16b(v):
    h = int(np.array([v], np.float16).view(np.uint16)[0])
    return [h & 0xFF, h >> 8]


def random_blocks(orc, t, n, seed):
    rng = np.random.default_rng(seed)
    ts = orc.TYPE_SIZE[t]
    raw = rng.integers(0, 256, size=ts * n, dtype=np.uint8)
    for b in range(n):
        o = b * ts
        if t in (Q8_0, Q4_0):
            raw[o:o + 2] = f16b(rng.uniform(-2, 2))
        elif t in (Q4_K, Q5_K):
            raw[o:o + 2] = f16b(rng.uniform(1e-4, 1e-1))
            raw[o + 2:o + 4] = f16b(rng.uniform(1e-4, 1e-1))
        elif t == Q6_K:
            raw[o + 208:o + 210] = f16b(rng.uniform(-1e-1, 1e-1))
    return raw


# --------------------------------------------------------------------------
# dequant: bit-exact
# --------------------------------------------------------------------------
def test_f16_widening_exhaustive(lrs, orc, ctx):
    codes = np.arange(65536, dtype=np.uint16)
    got = lrs.dequant_to_f32(ctx, F16, codes.view(np.uint8))
    ref = orc.dequant(F16, codes.view(np.uint8))
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), ref[~nan].view(np.uint32))


@pytest.mark.parametrize("t", [Q8_0, Q4_0, Q4_K, Q5_K, Q6_K, F32])
def test_dequant_bit_exact_random_blocks(lrs, orc, ctx, t):
    if t == F32:
        raw = np.random.default_rng(1).standard_normal(4096).astype(np.float32).view(np.uint8)
    else:
        raw = random_blocks(orc, t, 2048, 10 + t)
    got = lrs.dequant_to_f32(ctx, t, raw)
    ref = orc.dequant(t, raw)
    assert got.shape == ref.shape
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))


@pytest.mark.parametrize("t", KQ)
@pytest.mark.parametrize("mode", [0, 1])
def test_dequant_bit_exact_synthetic_blocks(lrs, orc, ctx, t, mode):
    raw = orc.gen_blocks(t, 1234 + t, 4096, mode=mode)
    got = lrs.dequant_to_f32(ctx, t, raw)
    assert np.array_equal(got.view(np.uint32), orc.dequant(t, raw).view(np.uint32))


def test_dequant_reference_known_answers(lrs, ctx):
    # dequant.rs:297-319, 366-394, 410-464 through the GPU
    out = lrs.dequant_to_f32(ctx, Q8_0, bytes(f16b(1.0) + [1, 0xFF] + [0] * 30))
    assert out[0] == 1.0 and out[1] == -1.0 and np.all(out[2:] == 0)
    out = lrs.dequant_to_f32(ctx, Q8_0, bytes(f16b(2.0) + [3] + [0] * 31))
    assert out[0] == 6.0
    out = lrs.dequant_to_f32(ctx, Q4_K, bytes(f16b(1.0) + f16b(1.0) + [8, 4] + [0] * 10 + [0x22] * 128))
    assert np.all(out[:32] == 16) and np.all(out[32:64] == 8) and np.all(out[64:] == 0)
    out = lrs.dequant_to_f32(ctx, Q6_K, bytes([0] * 192 + [1, 0] * 8 + f16b(1.0)))
    for base in (0, 128):
        for l in range(32):
            for off in (0, 32, 64, 96):
                assert out[base + l + off] == (-32.0 if l < 16 else 0.0)


def test_q5_k_gguf_py_golden_block_on_gpu(lrs, ctx):
    fx = json.load(open(os.path.join(HERE, "golden", "q5_k_gguf_py_block.json")))
    out = lrs.dequant_to_f32(ctx, Q5_K, bytes(fx["raw"]))
    for i, v in fx["spots"]:
        assert abs(out[i] - v) < fx["spot_tol"]
    assert abs(out.astype(np.float64).sum() - fx["sum"]) < fx["sum_tol"]


def test_dequant_rejects_bad_sizes(lrs, ctx):
    for t, bad in ((Q8_0, 33), (Q4_K, 143), (Q5_K, 175), (Q6_K, 209)):
        with pytest.raises(lrs.ModelError):
            lrs.dequant_to_f32(ctx, t, bytes(bad))


def test_read_probe_library_runs_and_rejects_bad_arguments(lrs, ctx):
    """liblrs_probe.so (the load-only read kernel behind bench.py --workload
    stream, kept out of liblrs.so) times reads in both load forms and refuses
    sizes that are not a multiple of 16, more than 4096 workgroups and thread
    counts that are not a multiple of 64 up to 1024, launching nothing."""
    import ctypes as C
    import os

    L = C.CDLL(os.path.join(os.path.dirname(lrs.LIB_PATH), "liblrs_probe.so"))
    L.lrsp_read_time.restype = C.c_int
    L.lrsp_read_time.argtypes = [C.c_int, C.c_void_p, C.c_size_t, C.c_uint32, C.c_int,
                                 C.c_uint32, C.c_uint32, C.c_uint32, C.c_int,
                                 C.POINTER(C.c_float)]
    buf = ctx.alloc(1 << 22)
    us = C.c_float()

    def run(window, nwin, nt, wg=0, th=0, reads=2, plain_first=0):
        return L.lrsp_read_time(0, buf.ptr, window, nwin, nt, wg, th, reads, plain_first,
                                C.byref(us))

    for nt in (0, 1):
        for wg in (0, 1, 512, 4096):
            assert run(1 << 20, 4, nt, wg) == 0 and us.value > 0
        assert run(4096 + 16, 1, nt) == 0
        assert run(1 << 20, 4, nt, 160, 768, 3, 1) == 0 and us.value > 0
    for th in (64, 1024):
        assert run(1 << 20, 4, 1, 160, th) == 0
    assert run(24, 1, 1) == -1
    assert run(1 << 20, 4, 1, 4097) == -1
    for th in (96, 1088):
        assert run(1 << 20, 4, 1, 160, th) == -1
    assert run(1 << 20, 0, 1) == -1 and run(1 << 20, 4, 1, reads=0) == -1
    ctx.sync()
    buf.free()


# --------------------------------------------------------------------------
# weights: upload / download / synthetic generator
# --------------------------------------------------------------------------
@pytest.mark.parametrize("t", KQ)
def test_upload_download_round_trip(lrs, orc, ctx, t):
    n_in = 512 if t != Q8_0 else 96
    raw = random_blocks(orc, t, 7 * n_in // orc.BLOCK[t], 5)
    w = lrs.Weight.upload(ctx, t, raw, n_in, 7)
    assert w.gguf_bytes == raw.nbytes
    assert np.array_equal(w.download(), raw)


@pytest.mark.parametrize("t", KQ)
@pytest.mark.parametrize("mode", [0, 1])
def test_device_generator_matches_host_generator(lrs, orc, ctx, t, mode):
    n_in, n_out = 1024, 33
    w = lrs.Weight.generate(ctx, t, 99 + t, n_in, n_out, mode=mode)
    ref = orc.gen_weight(t, 99 + t, n_out, n_in, mode=mode)
    assert np.array_equal(w.download(), ref)


def test_upload_rejects_bad_shapes(lrs, orc, ctx):
    raw = orc.gen_weight(Q4_K, 1, 4, 512)
    with pytest.raises(lrs.ModelError):
        lrs.Weight.upload(ctx, Q4_K, raw, 500, 4)  # n_in not a multiple of 256
    with pytest.raises(lrs.ModelError):
        lrs.Weight.upload(ctx, Q4_K, raw[:-1], 512, 4)  # wrong byte count
    with pytest.raises(lrs.ModelError):
        lrs.Weight.upload(ctx, 3, raw, 512, 4)  # Q4_1: not supported


# --------------------------------------------------------------------------
# matvec parity
# --------------------------------------------------------------------------
def ref_pattern_weights(t, n_in, n_out):
    """The reference's deterministic kernel-test weights (integration.rs:1115-1394)."""
    ts = {Q8_0: 34, Q4_K: 144, Q5_K: 176, Q6_K: 210}[t]
    nb = n_in // (32 if t == Q8_0 else 256)
    i = np.arange(n_out * nb * ts, dtype=np.int64)
    if t == Q8_0:
        w = ((i * 37) % 251).astype(np.uint8)
        w[i % 34 == 0] = 0x00
        w[i % 34 == 1] = 0x3C
        return w
    if t == Q6_K:
        w = ((i * 89 + i // 5) % 251).astype(np.uint8).reshape(-1, 210)
        w[:, 192:208] = np.array([((j * 7 % 40) - 20) for j in range(16)], np.int8).view(np.uint8)
        w[:, 208:210] = f16b(0.0091)
        return w.reshape(-1)
    w = ((i * 101 + i // 7) % 251).astype(np.uint8).reshape(-1, ts)
    w[:, 0:2] = f16b(0.0123)
    w[:, 2:4] = f16b(0.0045)
    return w.reshape(-1)


@pytest.mark.parametrize("t,n_in,n_out", [
    (Q4_K, 512, 16), (Q4_K, 4096, 16), (Q4_K, 5120, 16),
    (Q5_K, 512, 16), (Q5_K, 4096, 16), (Q5_K, 5120, 16),
    (Q6_K, 512, 16),
    (Q8_0, 4864, 64), (Q8_0, 5120, 64), (Q8_0, 13824, 64),
])
def test_matvec_reference_kernel_cases(lrs, orc, ctx, t, n_in, n_out):
    w = ref_pattern_weights(t, n_in, n_out)
    x = ((np.arange(n_in) % 29) - 14.0).astype(np.float32) * np.float32(0.031)
    got = lrs.Weight.upload(ctx, t, w, n_in, n_out).matvec(x)
    ref = orc.matvec(t, w, n_in, n_out, x)
    assert rel_l2(got, ref) < MATVEC_TOL
    assert np.abs(got - ref).max() / np.abs(ref).max() < 1e-5  # the reference's own bar




@pytest.mark.parametrize("t", KQ)
def test_matvec_every_geometry_ragged(lrs, orc, ctx, t):
    n_in = 1056 if t == Q8_0 else 1280  # unit count not a multiple of any lane count
    n_out = 37
    w = orc.gen_weight(t, 7, n_out, n_in, mode=1)
    x = orc.gen_normal(8, n_in)
    ref = orc.matvec(t, w, n_in, n_out, x)
    W = lrs.Weight.upload(ctx, t, w, n_in, n_out)
    try:
        for g in lrs.MATVEC_GEOMS:
            lrs.set_matvec_geom(*g)
            got = W.matvec(x)
            assert rel_l2(got, ref) < MATVEC_TOL, (g, rel_l2(got, ref))
    finally:
        lrs.set_matvec_geom(0, 0, 0)


@pytest.mark.parametrize("t", KQ)
def test_matvec_one_hot_selects_dequantized_column(lrs, orc, ctx, t):
    n_in, n_out = 512, 24
    w = orc.gen_weight(t, 3, n_out, n_in)
    deq = orc.dequant(t, w).reshape(n_out, n_in)
    W = lrs.Weight.upload(ctx, t, w, n_in, n_out)
    for col in (0, 33, 255, 256 + 77, n_in - 1):
        x = np.zeros(n_in, np.float32)
        x[col] = 1.0
        assert np.array_equal(W.matvec(x), deq[:, col])


@pytest.mark.parametrize("t", KQ)
def test_matvec_columns_equal_single_calls(lrs, orc, ctx, t):
    """integration.rs:1520-1577: a batched call equals per-column calls exactly."""
    n_in, n_out = 1024, 16
    w = orc.gen_weight(t, 4, n_out, n_in)
    W = lrs.Weight.upload(ctx, t, w, n_in, n_out)
    xs = np.stack([orc.gen_normal(20 + c, n_in) * (1 + c) for c in range(5)])
    yb = W.matvec(xs)
    for c in range(5):
        assert np.array_equal(yb[c], W.matvec(xs[c]))


# several columns per launch share each weight load (groups of 8, 4, 2, 1 as
# the LDS allows); every launch shape of the plain matvec appears
@pytest.mark.parametrize("t,n_in,n_out,cols", [
    (Q4_K, 1024, 16, 19), (Q8_0, 4096, 4096, 11), (Q6_K, 5120, 4096, 9),
    (Q5_K, 2048, 16384, 3), (Q4_K, 13824, 64, 5), (Q6_K, 768, 40, 8),
])
def test_matvec_columns_share_weight_loads_exactly(lrs, orc, ctx, t, n_in, n_out, cols):
    """Columns computed together equal the same columns one at a time and the
    staged form (pack launch + matvec launch) bit for bit, and the oracle to
    the matvec bar."""
    w = orc.gen_weight(t, 40 + cols, n_out, n_in)
    W = lrs.Weight.upload(ctx, t, w, n_in, n_out)
    xs = np.stack([orc.gen_normal(60 + c, n_in) * (1 + c % 3) for c in range(cols)])
    yb = W.matvec(xs)
    xd, yd = ctx.alloc(4 * n_in), ctx.alloc(4 * n_out)
    try:
        for c in range(cols):
            assert np.array_equal(yb[c], W.matvec(xs[c])), c
            xd.upload(xs[c])
            W.matvec_dev_noalloc(xd, yd)
            ctx.sync()
            assert np.array_equal(yb[c], yd.download(np.float32, n_out)), c
        ref = orc.matvec(t, w, n_in, n_out, xs, threads=THREADS)
        for c in range(cols):
            assert rel_l2(yb[c], ref[c]) < MATVEC_TOL, (c, rel_l2(yb[c], ref[c]))
    finally:
        xd.free()
        yd.free()


def test_matvec_zero_and_single_row(lrs, orc, ctx):
    for t in KQ:
        n_in = 256
        w = orc.gen_weight(t, 5, 1, n_in)
        x = orc.gen_normal(6, n_in)
        assert rel_l2(lrs.Weight.upload(ctx, t, w, n_in, 1).matvec(x),
                      orc.matvec(t, w, n_in, 1, x)) < MATVEC_TOL
    # all-zero quants: Q4_K gives -dmin * sum_j m_j * sum(x in j)
    raw = orc.gen_weight(Q4_K, 5, 8, 512).reshape(-1, 144)
    raw[:, 16:] = 0
    raw = raw.reshape(-1)
    x = orc.gen_normal(7, 512)
    assert rel_l2(lrs.Weight.upload(ctx, Q4_K, raw, 512, 8).matvec(x),
                  orc.matvec(Q4_K, raw, 512, 8, x)) < MATVEC_TOL


def test_matvec_rejects_unsupported(lrs, ctx):
    w = lrs.Weight.upload(ctx, F32, np.zeros(16, np.float32).view(np.uint8), 4, 4)
    with pytest.raises(lrs.ModelError):
        w.matvec(np.zeros(4, np.float32))
    w2 = lrs.Weight.generate(ctx, Q4_K, 1, 256, 4)
    with pytest.raises(lrs.ModelError):
        w2.matvec(np.zeros(255, np.float32))


# BASELINE configs 1 and 2 at full size, BASELINE distributions
CFG1 = [("q8_0", Q8_0, 4096, 4096)]
CFG2 = [("attn_q", Q4_K, 5120, 5120), ("attn_k", Q4_K, 5120, 1024),
        ("attn_v", Q6_K, 5120, 1024), ("attn_output", Q4_K, 5120, 5120),
        ("ffn_gate", Q4_K, 5120, 13824), ("ffn_up", Q4_K, 5120, 13824),
        ("ffn_down", Q6_K, 13824, 5120)]


@pytest.mark.parametrize("name,t,n_in,n_out", CFG1 + CFG2)
def test_matvec_baseline_config_shapes(lrs, orc, ctx, name, t, n_in, n_out):
    seed = 1000 + n_in + n_out + t
    W = lrs.Weight.generate(ctx, t, seed, n_in, n_out)
    host = orc.gen_weight(t, seed, n_out, n_in)
    x = orc.gen_normal(1234, n_in)
    got = W.matvec(x)
    ref = orc.matvec(t, host, n_in, n_out, x, threads=THREADS)
    assert rel_l2(got, ref) < MATVEC_TOL, rel_l2(got, ref)


def test_captured_graph_replays_match_eager(lrs, orc, ctx):
    """lrs_capture_begin/end + lrs_graph_launch: two matvecs and a GEMM recorded
    once, replayed three times with eager work and synchronisations between
    the replays; every replay equals the eager result bit for bit."""
    n_in, n_out, m = 1024, 512, 64
    wa = lrs.Weight.upload(ctx, 12, orc.gen_weight(12, 71, n_out, n_in, mode=1), n_in, n_out)
    wb = lrs.Weight.upload(ctx, 14, orc.gen_weight(14, 72, n_out, n_in, mode=1), n_in, n_out)
    rng = np.random.default_rng(3)
    x = ctx.alloc(4 * n_in * m)
    x.upload(rng.standard_normal(n_in * m).astype(np.float32))
    ya, yb, yg = ctx.alloc(4 * n_out), ctx.alloc(4 * n_out), ctx.alloc(4 * n_out * m)

    def work():
        wa.matvec_dev(x, ya)
        wb.matvec_dev(x, yb)
        wa.gemm_dev(x, yg, m, precision=3)

    work()  # eager (also sizes the context scratch outside the capture)
    ctx.sync()
    want = [b.download(np.float32, k) for b, k in ((ya, n_out), (yb, n_out), (yg, n_out * m))]
    g = ctx.capture(work)
    for rep in range(3):
        for b in (ya, yb, yg):
            b.upload(np.full(b.nbytes // 4, np.nan, np.float32))
        g.launch()
        ctx.sync()
        got = [b.download(np.float32, k) for b, k in ((ya, n_out), (yb, n_out), (yg, n_out * m))]
        for a, b in zip(got, want):
            assert np.array_equal(a, b), rep
        wb.matvec_dev(x, ya)  # eager work between the replays
        ctx.sync()
    g.close()


def test_scratch_growth_refused_while_a_graph_lives(lrs, orc):
    """A graph records the context scratch address: a call that would grow
    the scratch while the graph is alive fails (LRS_E_ARG) and leaves the
    buffer in place, so the graph still replays correctly; once the graph is
    destroyed the same call succeeds."""
    c = lrs.Context(0)
    try:
        # one Q4_K column wider than 4096: the staged form, whose input pack
        # lives in the context scratch (sized here, outside the capture)
        n_in, n_out = 8192, 256
        w = lrs.Weight.upload(c, Q4_K, orc.gen_weight(Q4_K, 81, n_out, n_in, mode=1), n_in, n_out)
        x = c.alloc(4 * n_in)
        x.upload(orc.gen_normal(82, n_in))
        y = c.alloc(4 * n_out)
        w.matvec_dev(x, y)
        c.sync()
        want = y.download(np.float32, n_out)
        g = c.capture(lambda: w.matvec_dev(x, y))
        # a GEMM whose bf16 operand planes need more than the current scratch
        m = 1024
        big = lrs.Weight.upload(c, Q4_K, orc.gen_weight(Q4_K, 83, 256, 4096, mode=1), 4096, 256)
        a = c.alloc(4 * m * 4096)
        yg = c.alloc(4 * m * 256)
        with pytest.raises(lrs.ModelError) as e:
            big.gemm_dev(a, yg, m, precision=3)
        assert e.value.code == -1 and "graph" in str(e.value)
        # had the scratch been freed, memory allocated now could take its
        # address and the replay (which writes the pack there) would overwrite it
        guards = [c.alloc(1 << 20) for _ in range(4)]
        pattern = np.arange(1 << 18, dtype=np.uint32)
        for b in guards:
            b.upload(pattern)
        y.upload(np.full(n_out, np.nan, np.float32))
        g.launch()
        c.sync()
        assert np.array_equal(y.download(np.float32, n_out), want)
        for b in guards:
            assert np.array_equal(b.download(np.uint32, 1 << 18), pattern)
            b.free()
        g.close()
        a.upload(np.zeros(m * 4096, np.float32))
        big.gemm_dev(a, yg, m, precision=3)  # grows now
        c.sync()
        assert not np.any(yg.download(np.float32, m * 256))
    finally:
        c.close()


# --------------------------------------------------------------------------
# int8-activation Q8_0 path (ops.rs:284-385, 704-724, 728-886)
# --------------------------------------------------------------------------
def q8_inputs(seed):
    """normal data, blocks with exact ties (max 127 * 2^s), a zero block, an
    f16-underflowing block and a large block"""
    rng = np.random.default_rng(seed)
    x = rng.standard_normal(32 * 512).astype(np.float32)
    for b in range(0, 64):
        s = int(rng.integers(-30, 20))
        k = rng.integers(-127, 128, size=32) + np.where(rng.random(32) < 0.5, 0.5, 0.0)
        k = np.clip(k, -127, 127)
        k[0] = 127
        x[32 * b:32 * b + 32] = (k * 2.0 ** s).astype(np.float32)
    x[32 * 64:32 * 65] = 0.0
    x[32 * 65:32 * 66] *= np.float32(2.0 ** -45)
    x[32 * 66:32 * 67] *= np.float32(1e30)
    return x


@pytest.mark.parametrize("half_even", [True, False])
def test_q8_quantize_bit_exact(lrs, orc, ctx, half_even):
    x = q8_inputs(3)
    got = lrs.quantize_q8_0(ctx, x, half_even)
    ref = orc.quantize_q8_0(x, half_even)
    assert np.array_equal(got, ref)


@pytest.mark.parametrize("n_in,n_out", [(32, 2), (1056, 37), (4096, 4096), (13824, 64)])
@pytest.mark.parametrize("half_even", [True, False])
def test_q8_actq_matvec_matches_oracle(lrs, orc, ctx, n_in, n_out, half_even):
    w = orc.gen_weight(Q8_0, 21, n_out, n_in)
    x = orc.gen_normal(22, n_in) * np.float32(3.0)
    got = lrs.Weight.upload(ctx, Q8_0, w, n_in, n_out).matvec_actq(x, half_even)
    ref = orc.matvec_q8_0_actq(w, n_in, n_out, x, half_even)
    assert rel_l2(got, ref) < MATVEC_TOL


def test_q8_actq_reference_fixture_exact(lrs, ctx):
    """ops.rs:1212-1245 fixture: y = [20 f16(32/127), 8 f16(32/127)] exactly."""
    w = np.array(f16b(1.0) + [1, 2] + [0] * 30 + f16b(2.0) + [1] + [0] * 31, np.uint8)
    x = np.arange(1, 33, dtype=np.float32)
    y = lrs.Weight.upload(ctx, Q8_0, w, 32, 2).matvec_actq(x)
    assert y.tolist() == [5.0390625, 2.015625]


def test_q8_actq_columns_and_errors(lrs, orc, ctx):
    n_in, n_out = 512, 16
    w = orc.gen_weight(Q8_0, 23, n_out, n_in)
    W = lrs.Weight.upload(ctx, Q8_0, w, n_in, n_out)
    xs = np.stack([orc.gen_normal(30 + c, n_in) for c in range(3)])
    yb = W.matvec_actq(xs)
    for c in range(3):
        assert np.array_equal(yb[c], W.matvec_actq(xs[c]))
    w4 = orc.gen_weight(Q4_K, 24, n_out, n_in)
    with pytest.raises(lrs.ModelError):
        lrs.Weight.upload(ctx, Q4_K, w4, n_in, n_out).matvec_actq(xs[0])
    with pytest.raises(lrs.ModelError):
        lrs.quantize_q8_0(ctx, np.ones(33, np.float32))
