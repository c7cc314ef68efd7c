"""Results written by one launch and read back by the next kernel while the
L2 may still hold the previous contents of the same lines.

The fixed-order average and AdamW stream their outputs with non-temporal
stores, and the DDP average writes each merged run of buckets as a slice of
one flat buffer, so run boundaries fall inside cache lines. A kernel that
reads the buffer right afterwards (the norm pass, the next average's caller)
must see every element of the new values, over many rounds in which the
previous round's values were just read on the GPU."""
import numpy as np
import pytest

from helpers import bits_equal

pytestmark = pytest.mark.gpu


def _dev():
    from dtmi import device as D, kernels as K
    return D, K


@pytest.mark.parametrize("dt", [np.float32, np.float64])
def test_average_slices_read_back_after_each_round(dev, dt):
    D, K = _dev()
    n, W = 4099, 4
    # run boundaries inside cache lines: 16-byte aligned (the vector path) and not
    cuts = [0, 4, 36, 300, 1028, 1111, 2052, 3001, 4099]
    rows = D.empty((W, n), dt)
    out = D.empty((n,), dt)
    sq = D.empty((1,), np.float64)
    rng = np.random.default_rng(11)
    for it in range(24):
        r = rng.standard_normal((W, n)).astype(dt)
        rows.assign(r)
        for lo, hi in zip(cuts[:-1], cuts[1:]):
            cols = D.DeviceArray(rows.block, (W, hi - lo), rows.dtype, rows.offset + lo * rows.itemsize,
                                 (rows.strides[0], 1))
            K.bucket_average(out[lo:hi], cols, W, 1.0 / W)
        K.sumsq([out], sq)  # reads every line of `out` on the GPU
        exp = ((r[0] + r[1]) + r[2]) + r[3]
        exp = exp * dt(1.0 / W)
        want = float(np.dot(exp.astype(np.float64), exp.astype(np.float64)))
        assert abs(sq.numpy()[0] - want) <= 1e-12 * want, it
        assert bits_equal(out.numpy(), exp), it


@pytest.mark.parametrize("dt", [np.float32, np.float64])
def test_adamw_shard_slices_read_back_after_each_round(dev, dt):
    """AdamW over sub-ranges of one flat buffer whose boundaries fall inside
    cache lines, the parameters read back on the GPU (sum of squares) after
    every step and compared with the oracle's update."""
    from oracle import optim as OO
    D, K = _dev()
    n = 3001
    cuts = [0, 4, 36, 999, 1028, 2052, 3001]
    rng = np.random.default_rng(12)
    p = (rng.standard_normal(n) * 0.02).astype(dt)
    m = np.abs(rng.standard_normal(n) * 1e-4).astype(dt)
    v = np.abs(rng.standard_normal(n) * 1e-4).astype(dt)
    dp, dm, dv = D.from_numpy(p), D.from_numpy(m), D.from_numpy(v)
    sq = D.empty((1,), np.float64)
    for t in range(1, 13):
        g = (rng.standard_normal(n) * 1e-3).astype(dt)
        dg = D.from_numpy(g)
        b1t, b2t = 1 - 0.9 ** t, 1 - 0.95 ** t
        for lo, hi in zip(cuts[:-1], cuts[1:]):
            K.adamw(dp[lo:hi], dg[lo:hi], dm[lo:hi], dv[lo:hi], 3e-4, 0.9, 0.95, 1e-8, 0.1, b1t, b2t)
        K.sumsq([dp], sq)
        OO.adamw_update(p, g, m, v, 3e-4, 0.9, 0.95, 1e-8, 0.1, b1t, b2t)
        want = float(np.dot(p.astype(np.float64), p.astype(np.float64)))
        assert abs(sq.numpy()[0] - want) <= 1e-12 * want, t
        assert bits_equal(dp.numpy(), p), t
