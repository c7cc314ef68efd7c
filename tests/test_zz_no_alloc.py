"""dtmi_layernorm_bwd_noalloc, the LayerNorm backward that allocates nothing
(its column partials live in a fixed device array), against
dtmi_layernorm_bwd through the C ABI: the same dx, dgamma and dbeta bits on
two calls in a row, the second with a smaller input; no pool memory taken;
oversized shapes refused before any launch."""
import ctypes

import numpy as np
import pytest

from helpers import bits_equal

pytestmark = pytest.mark.gpu


def _setup(rng, rows, cols, dt):
    from dtmi import device as D, kernels as K
    x = D.from_numpy(rng.standard_normal((rows, cols)).astype(dt))
    w = D.from_numpy((1 + 0.01 * rng.standard_normal(cols)).astype(dt))
    b = D.from_numpy((0.01 * rng.standard_normal(cols)).astype(dt))
    dy = D.from_numpy(rng.standard_normal((rows, cols)).astype(dt))
    _, mean, rstd = K.layernorm_fwd(x, w, b)
    return x, w, dy, mean, rstd


def _outs(x, dt):
    from dtmi import device as D
    rows, cols = x.shape
    return D.full((rows, cols), 3.0, dt), D.full((cols,), 5.0, dt), D.full((cols,), 7.0, dt)


def _call(name, dt, x, w, dy, mean, rstd, accumulate=0, outs=None):
    from dtmi import _lib
    rows, cols = x.shape
    if outs is None:
        outs = _outs(x, dt)
    dx, dw, db = outs
    rc = getattr(_lib.lib(), name)(_lib.dtype_code(dt), dx.ptr, dw.ptr, db.ptr, dy.ptr, x.ptr, w.ptr, mean.ptr,
                                   rstd.ptr, rows, cols, accumulate)
    return rc, outs


def _stats():
    from dtmi import _lib
    return _lib.memory_stats()


@pytest.mark.parametrize("dt", [np.float32, np.float64])
def test_noalloc_layernorm_backward_matches_the_pooled_entry_point(dev, dt):
    from dtmi import _lib
    rng = np.random.default_rng(99)
    # first a GPT-2-small LayerNorm (8192 x 768), then a smaller one (ragged,
    # fewer partial rows): the array keeps the first call's partials, which
    # the second call must overwrite where it reads them
    for rows, cols in ((8192, 768), (37, 100)):
        if dt == np.float64 and cols == 768:
            rows = 4096
        args = _setup(rng, rows, cols, dt)
        rc, ref = _call("dtmi_layernorm_bwd", dt, *args)
        assert rc == 0
        outs = _outs(args[0], dt)
        _lib.sync()
        before = _stats()
        rc, got = _call("dtmi_layernorm_bwd_noalloc", dt, *args, outs=outs)
        assert rc == 0, _lib.lib().dtmi_last_error()
        _lib.sync()
        after = _stats()
        # outputs were made before the call; the call itself takes no pool memory
        assert after["in_use"] == before["in_use"] and after["cached"] == before["cached"]
        for a, r in zip(got, ref):
            assert bits_equal(a.numpy(), r.numpy())
        # accumulate bits: dx += and dgamma/dbeta +=
        rc, ref2 = _call("dtmi_layernorm_bwd", dt, *args, accumulate=3, outs=ref)
        assert rc == 0
        rc, got2 = _call("dtmi_layernorm_bwd_noalloc", dt, *args, accumulate=3, outs=got)
        assert rc == 0
        for a, r in zip(got2, ref2):
            assert bits_equal(a.numpy(), r.numpy())


def test_noalloc_layernorm_backward_refuses_shapes_beyond_its_array(dev):
    """float32 rows of 4096 columns at 4096 rows need 16 MiB of partials: refused
    with a message, and nothing written."""
    from dtmi import _lib, device as D
    rows, cols = 4096, 4096
    x = D.zeros((rows, cols), np.float32)
    w = D.full((cols,), 1.0, np.float32)
    mean, rstd = D.zeros((rows,), np.float32), D.full((rows,), 1.0, np.float32)
    dx = D.full((rows, cols), 2.0, np.float32)
    dw, db = D.full((cols,), 2.0, np.float32), D.full((cols,), 2.0, np.float32)
    rc = _lib.lib().dtmi_layernorm_bwd_noalloc(_lib.F32, dx.ptr, dw.ptr, db.ptr, x.ptr, x.ptr, w.ptr, mean.ptr,
                                               rstd.ptr, rows, cols, 0)
    assert rc == 1
    assert b"scratch" in _lib.lib().dtmi_last_error()
    _lib.sync()
    assert np.all(dw.numpy() == 2.0) and np.all(dx.numpy()[:2] == 2.0)
    # the same shape through the pooled entry point works
    rc = _lib.lib().dtmi_layernorm_bwd(_lib.F32, dx.ptr, dw.ptr, db.ptr, x.ptr, x.ptr, w.ptr, mean.ptr, rstd.ptr,
                                       rows, cols, 0)
    assert rc == 0
    _lib.sync()
    assert ctypes.sizeof(ctypes.c_float) == 4
