"""Empty inputs through the C ABI: NumPy's semantics (an empty product is
zeros, a sum over no rows is zero), no launch on an empty grid, no error."""
import numpy as np
import pytest

from helpers import bits_equal

pytestmark = pytest.mark.gpu


def _dev():
    from dtmi import device as D, kernels as K
    return D, K


@pytest.mark.parametrize("dt", [np.float32, np.float64])
def test_empty_inputs(dev, dt):
    D, K = _dev()
    z = lambda *s: D.from_numpy(np.zeros(s, dt))  # noqa: E731
    one = lambda *s: D.from_numpy(np.ones(s, dt))  # noqa: E731
    # elementwise and the column sum over no rows
    a, b = z(0, 5), z(0, 5)
    assert K.binary("add", a, b).shape == (0, 5)
    assert K.gelu_fwd(a).shape == (0, 5)
    assert K.scale(a, 2.0).shape == (0, 5)
    assert bits_equal(K.colsum(a).numpy(), np.zeros(5, dt))
    # products with an empty dimension: M = 0, N = 0, and K = 0 (zeros)
    assert K.gemm(one(0, 4), one(4, 3)).shape == (0, 3)
    assert K.gemm(one(2, 4), one(4, 0)).shape == (2, 0)
    assert bits_equal(K.gemm(one(2, 0), one(0, 3)).numpy(), np.zeros((2, 3), dt))
    assert bits_equal(K.gemm(one(2, 0), one(0, 3), bias=D.from_numpy(np.arange(3, dtype=dt))).numpy(),
                      np.tile(np.arange(3, dtype=dt), (2, 1)))
    # LayerNorm over no rows: empty outputs, zero dgamma and dbeta
    x, w, bb = z(0, 8), one(8), z(8)
    y, mean, rstd = K.layernorm_fwd(x, w, bb)
    assert y.shape == (0, 8) and mean.shape == (0,)
    dx, dw, db = K.layernorm_bwd(z(0, 8), x, w, mean, rstd)
    assert dx.shape == (0, 8)
    assert bits_equal(dw.numpy(), np.zeros(8, dt)) and bits_equal(db.numpy(), np.zeros(8, dt))
    # attention with no queries and with no batch elements
    for shape in ((1, 2, 0, 16), (0, 2, 8, 16)):
        q, k, v, g = (z(*shape) for _ in range(4))
        o, rmax, rsum = K.attn_fwd(q, k, v)
        assert o.shape == shape
        for t in K.attn_bwd(q, k, v, o, g, rmax, rsum):
            assert t.shape == shape
    # the gradient path on no elements: average, AdamW, sum of squares
    out = z(0)
    K.bucket_average(out, z(4, 0), 4, 0.25)
    p, g, m, vv = z(0), z(0), z(0), z(0)
    K.adamw(p, g, m, vv, 1e-3, 0.9, 0.95, 1e-8, 0.1, 0.1, 0.05)
    sq = D.from_numpy(np.full(1, 7.0))
    K.sumsq([z(0)], sq)
    assert sq.numpy()[0] == 0.0
