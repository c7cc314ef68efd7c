"""Generic tensor-op kernels on the GPU against the oracle / NumPy.

IEEE add/sub/mul and copies are bit-exact; GELU (device tanh) is within
1e-12 (float64) / 1e-5 (float32) normwise; reductions are within tolerance and
deterministic.
"""
import numpy as np
import pytest

from helpers import bits_equal, rel_err
from oracle import ops

pytestmark = pytest.mark.gpu


def _dev():
    from dtmi import device as D, kernels as K
    return D, K


@pytest.mark.parametrize("dt", [np.float64, np.float32])
def test_binary_broadcast_exact(dev, dt):
    D, K = _dev()
    rng = np.random.default_rng(0)
    for sa, sb in [((3, 4), (4,)), ((2, 3, 4), (1, 4)), ((3, 1), (3, 5)), ((64, 3072), (3072,)), ((5,), (5,)),
                   ((2, 1, 3), (4, 1)), ((), ())]:
        a = rng.standard_normal(sa).astype(dt)
        b = rng.standard_normal(sb).astype(dt)
        for op, f in (("add", np.add), ("sub", np.subtract), ("mul", np.multiply)):
            got = K.binary(op, D.from_numpy(a), D.from_numpy(b)).numpy()
            assert bits_equal(got, f(a, b).astype(dt)), (op, sa, sb)


def test_strided_copy_exact(dev):
    D, K = _dev()
    rng = np.random.default_rng(1)
    x = rng.standard_normal((2, 5, 3, 4, 6)).astype(np.float32)
    dx = D.from_numpy(x)
    t = dx.transpose(2, 0, 3, 1, 4)
    assert not t.is_contiguous
    assert bits_equal(t.numpy(), x.transpose(2, 0, 3, 1, 4))
    assert bits_equal(t.reshape(3, -1).numpy(), x.transpose(2, 0, 3, 1, 4).reshape(3, -1))
    y = D.zeros((6, 4, 3, 5, 2), np.float32)
    y.transpose(4, 3, 2, 1, 0).assign(dx)
    assert bits_equal(y.numpy(), x.transpose(4, 3, 2, 1, 0))


@pytest.mark.parametrize("dt,tol", [(np.float64, 1e-12), (np.float32, 1e-5)])
def test_gelu_forward_backward(dev, dt, tol):
    D, K = _dev()
    rng = np.random.default_rng(2)
    x = (rng.standard_normal(1_000_003) * 3).astype(dt)
    g = rng.standard_normal(x.size).astype(dt)
    y, t, c = ops.gelu_fwd(x)
    dx = ops.gelu_bwd(g, x, t, c)
    dxd = D.from_numpy(x)
    assert rel_err(K.gelu_fwd(dxd).numpy(), y) <= tol
    assert rel_err(K.gelu_bwd(dxd, D.from_numpy(g)).numpy(), dx) <= tol


def test_relu_exact(dev):
    D, K = _dev()
    x = np.random.default_rng(3).standard_normal(1000)
    g = np.random.default_rng(4).standard_normal(1000)
    y, m = ops.relu_fwd(x)
    assert bits_equal(K.relu_fwd(D.from_numpy(x)).numpy(), y)
    assert bits_equal(K.relu_bwd(D.from_numpy(x), D.from_numpy(g)).numpy(), ops.relu_bwd(g, m))


@pytest.mark.parametrize("dt", [np.float64, np.float32])
@pytest.mark.parametrize("shape,axes", [((8, 1024, 768), [0]), ((19, 6, 20), [0]), ((3, 5, 7, 8), [0, 1]),
                                        ((10, 7), [0]), ((4, 9, 3), [0])])
def test_reduce_leading_axes_bit_exact(dev, dt, shape, axes):
    """Sums over leading axes (the position-embedding gradient's batch sum)
    add the reduced rows in ascending order, vector path or not: the bits of
    an explicit row-by-row sum."""
    D, K = _dev()
    x = np.random.default_rng(len(shape) * 31 + shape[0]).standard_normal(shape).astype(dt)
    nred = int(np.prod([shape[a] for a in axes]))
    rows = x.reshape(nred, -1)
    ref = np.zeros(rows.shape[1], dt)
    for r in range(nred):
        ref = ref + rows[r]
    got = K.reduce_sum(D.from_numpy(x), axes).numpy()
    assert bits_equal(got.reshape(-1), ref)


@pytest.mark.parametrize("dt,tol", [(np.float64, 1e-13), (np.float32, 1e-5)])
def test_reductions(dev, dt, tol):
    D, K = _dev()
    rng = np.random.default_rng(5)
    x = rng.standard_normal((3, 4, 2, 5)).astype(dt)
    for axes in ([0], [1], [0, 2], [3], [0, 1, 2, 3]):
        got = K.reduce_sum(D.from_numpy(x), axes).numpy()
        assert rel_err(got, x.sum(axis=tuple(axes))) <= tol
    big = rng.standard_normal((8192, 3072)).astype(dt)
    d = D.from_numpy(big)
    a = K.colsum(d).numpy()
    b = K.colsum(d).numpy()
    assert bits_equal(a, b)
    assert rel_err(a, ops.unbroadcast(big, (3072,))) <= tol
