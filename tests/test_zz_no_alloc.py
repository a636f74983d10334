"""lrs_matvec_dev_noalloc (static device pack, no allocation) against
lrs_matvec_dev (context scratch) through the C ABI: identical kernels and
pack, so the outputs must be identical, on two calls in a row, the second
with a smaller input."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu
Q8_0, Q4_K, Q6_K = 8, 12, 14


def _case(lrs, orc, ctx, t, n_in, n_out, cols, seed):
    w = lrs.Weight.upload(ctx, t, orc.gen_weight(t, seed, n_out, n_in, mode=1), n_in, n_out)
    x = ctx.alloc(4 * n_in * cols)
    x.upload(orc.gen_normal(seed + 1, n_in * cols))
    ya, yb = ctx.alloc(4 * n_out * cols), ctx.alloc(4 * n_out * cols)
    ya.upload(np.full(n_out * cols, np.nan, np.float32))
    yb.upload(np.full(n_out * cols, np.nan, np.float32))
    w.matvec_dev(x, ya, cols)
    w.matvec_dev_noalloc(x, yb, cols)
    ctx.sync()
    a, b = ya.download(np.float32, n_out * cols), yb.download(np.float32, n_out * cols)
    assert not np.any(np.isnan(a))
    assert np.array_equal(a, b), (t, n_in, n_out)
    ref = orc.matvec(t, orc.gen_weight(t, seed, n_out, n_in, mode=1), n_in, n_out,
                     orc.gen_normal(seed + 1, n_in * cols).reshape(cols, n_in), threads=8)
    err = np.linalg.norm(b - ref.ravel()) / np.linalg.norm(ref)
    assert err < 1e-4, err


def test_noalloc_matvec_matches_scratch_matvec(lrs, orc):
    c = lrs.Context(0)
    try:
        # the largest input the static pack holds, then a smaller one
        _case(lrs, orc, c, Q4_K, lrs.NOALLOC_MAX_N_IN, 96, 1, 31)
        _case(lrs, orc, c, Q6_K, 2560, 160, 2, 33)
        _case(lrs, orc, c, Q8_0, 4096, 64, 1, 35)
    finally:
        c.close()


def test_noalloc_matvec_rejects_inputs_beyond_the_static_pack(lrs, orc):
    c = lrs.Context(0)
    try:
        n_in = lrs.NOALLOC_MAX_N_IN + 256
        w = lrs.Weight.upload(c, Q4_K, orc.gen_weight(Q4_K, 41, 16, n_in, mode=1), n_in, 16)
        x, y = c.alloc(4 * n_in), c.alloc(4 * 16)
        with pytest.raises(lrs.ModelError) as e:
            w.matvec_dev_noalloc(x, y)
        assert e.value.code == -1
    finally:
        c.close()
