"""GPU parity of the batched-prefill dequant-GEMM (lrs_gemm_dev) against the
CPU oracle's dequant (bit-exact dequant.rs restatement) and float64 products.

precision 1 (bf16 operands, f32 accumulation) is checked
against the exact product of the same bf16-rounded operands (tolerance 1e-5
relative L2: only the f32 summation order differs); precision 3 (bf16 hi/lo
split) against the f32 operands themselves (tolerance 1e-4, the north-star
GEMM bar).
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu
Q8_0, Q4_K, Q5_K, Q6_K = 8, 12, 13, 14


@pytest.fixture(scope="module")
def ctx(lrs):
    c = lrs.Context(0)
    yield c
    c.close()


def bf16(x):
    """Round float32 to the nearest bfloat16 (ties to even), as float32."""
    b = np.ascontiguousarray(x, np.float32).view(np.uint32).astype(np.uint64)
    b = (b + 0x7FFF + ((b >> 16) & 1)) & 0xFFFF0000
    return b.astype(np.uint32).view(np.float32)


def rel_l2(a, b):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / np.linalg.norm(b))


@pytest.mark.parametrize("t", [Q4_K, Q5_K, Q6_K, Q8_0])
# (64, 256, 4096), (96, 128, 8192) and (512, 384, 4096) split K over
# workgroups (few output tiles, long K); m >= 512 uses the 256-token tile at
# precision 1 (ragged m and n included)
@pytest.mark.parametrize("m,n,k", [(1, 200, 512), (7, 128, 256), (130, 300, 768), (256, 256, 1024),
                                   (64, 256, 4096), (96, 128, 8192), (512, 256, 1024),
                                   (600, 200, 512), (512, 384, 4096), (1000, 136, 2048)])
def test_gemm_matches_oracle(lrs, orc, ctx, t, m, n, k):
    w = orc.gen_weight(t, 31 + m + n, n, k, mode=1)
    deq = orc.dequant(t, w).reshape(n, k)
    a = np.random.default_rng(m * 7 + n).standard_normal((m, k)).astype(np.float32)
    W = lrs.Weight.upload(ctx, t, w, k, n)
    y1 = W.gemm(a, precision=1)
    ref1 = bf16(a).astype(np.float64) @ bf16(deq).astype(np.float64).T
    assert rel_l2(y1, ref1) < 1e-5
    y3 = W.gemm(a, precision=3)
    ref = a.astype(np.float64) @ deq.astype(np.float64).T
    assert rel_l2(y3, ref) < 1e-4
    # plain bf16 is ~2^-9 per operand: far from f32, which is why prefill uses 3
    assert rel_l2(y1, ref) < 1e-2


def test_gemm_row_of_one_hot_activations_is_a_weight_column(lrs, orc, ctx):
    """a = identity rows: y[i] = column i of W (exact for values that bf16
    represents, which the hi/lo split reaches to 2^-16)."""
    k, n = 256, 64
    w = orc.gen_weight(Q4_K, 5, n, k, mode=1)
    deq = orc.dequant(Q4_K, w).reshape(n, k)
    a = np.eye(k, dtype=np.float32)[:40]
    y = lrs.Weight.upload(ctx, Q4_K, w, k, n).gemm(a, precision=3)
    assert np.allclose(y, deq[:, :40].T, rtol=2e-5, atol=0)


def test_gemm_rejects_bad_arguments(lrs, orc, ctx):
    # n_in must be a multiple of 256 (one K-step of the tile), for Q8_0 too
    w = lrs.Weight.upload(ctx, Q8_0, orc.gen_weight(Q8_0, 1, 4, 64), 64, 4)
    with pytest.raises(lrs.ModelError):
        w.gemm(np.zeros((2, 64), np.float32))
    w4 = lrs.Weight.upload(ctx, Q4_K, orc.gen_weight(Q4_K, 1, 4, 256), 256, 4)
    with pytest.raises(lrs.ModelError):
        w4.gemm(np.zeros((2, 256), np.float32), precision=2)


@pytest.mark.parametrize("types,m", [((Q4_K, Q4_K, Q6_K), 512), ((Q4_K, Q4_K, Q6_K), 130),
                                     ((Q5_K, Q6_K), 600), ((Q8_0, Q8_0), 77), ((Q6_K,), 256)])
def test_gemm_group_equals_single_gemms(lrs, orc, ctx, types, m):
    """lrs_gemm_group_dev (the prompt block's q / k / v as one launch, segments
    of ragged width and two types) against the oracle at both precisions and
    against one lrs_gemm_dev call per weight (the same per-tile arithmetic;
    the single calls may split K, so within 1e-6 rather than bit-exact)."""
    k = 1024
    widths = [200, 136, 72][:len(types)]
    ws, deqs = [], []
    for i, (t, n) in enumerate(zip(types, widths)):
        w = orc.gen_weight(t, 71 + i, n, k, mode=1)
        deqs.append(orc.dequant(t, w).reshape(n, k))
        ws.append(lrs.Weight.upload(ctx, t, w, k, n))
    a = np.random.default_rng(m).standard_normal((m, k)).astype(np.float32)
    for prec in (1, 3):
        ys = lrs.gemm_group(ctx, ws, a, precision=prec)
        for y, w, deq in zip(ys, ws, deqs):
            single = w.gemm(a, precision=prec)
            assert rel_l2(y, single) < 1e-6
            if prec == 3:
                ref = a.astype(np.float64) @ deq.astype(np.float64).T
                assert rel_l2(y, ref) < 1e-4
            else:
                ref = bf16(a).astype(np.float64) @ bf16(deq).astype(np.float64).T
                assert rel_l2(y, ref) < 1e-5


def test_gemm_group_rejects_bad_groups(lrs, orc, ctx):
    w4 = lrs.Weight.upload(ctx, Q4_K, orc.gen_weight(Q4_K, 1, 16, 512), 512, 16)
    w6 = lrs.Weight.upload(ctx, Q6_K, orc.gen_weight(Q6_K, 2, 16, 512), 512, 16)
    w8 = lrs.Weight.upload(ctx, Q8_0, orc.gen_weight(Q8_0, 3, 16, 512), 512, 16)
    w4k = lrs.Weight.upload(ctx, Q4_K, orc.gen_weight(Q4_K, 4, 16, 256), 256, 16)
    a = np.zeros((4, 512), np.float32)
    for group in ([w6, w4], [w4, w6, w4], [w4, w8], [w4, w4k], [w4, w4, w4, w4]):
        with pytest.raises(lrs.ModelError):
            lrs.gemm_group(ctx, group, a)
