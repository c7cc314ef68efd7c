"""Bandwidth kernels (LayerNorm, cross entropy, softmax backward, embedding) and
the MFMA GEMM on the GPU against the oracle.

Bar: float64 normwise relative error <= 1e-12, float32 <= 1e-5; the embedding
backward is bit-exact (same additions in the same order as np.add.at);
reductions are deterministic (two runs, same bits).
"""
import numpy as np
import pytest

from helpers import bits_equal, rel_err
from oracle import ops

pytestmark = pytest.mark.gpu

TOL = {np.float64: 1e-12, np.float32: 1e-5}


def _dev():
    from dtmi import device as D, kernels as K
    return D, K


@pytest.mark.parametrize("dt", [np.float64, np.float32])
@pytest.mark.parametrize("shape", [(2, 3, 6), (256, 64), (4096, 768), (5, 1000), (3, 17), (2400, 1000), (5000, 768),
                                   (33, 2000), (9, 2048), (3, 1025), (7, 5000), (130, 2304), (2, 70001), (600, 4097)])
def test_layernorm_forward_backward(dev, dt, shape):
    """Rows in registers (up to 16 vectors per lane) and longer rows (a block
    per row: unaligned rows above 1024, float64 above 2048, float32 above
    4096 elements)."""
    D, K = _dev()
    rng = np.random.default_rng(sum(shape))
    C = shape[-1]
    x = rng.standard_normal(shape).astype(dt)
    w = (1 + 0.01 * rng.standard_normal(C)).astype(dt)
    b = (0.01 * rng.standard_normal(C)).astype(dt)
    g = rng.standard_normal(shape).astype(dt)
    y, cache = ops.layer_norm_fwd(x, w, b)
    gx, gw, gb = ops.layer_norm_bwd(g, cache, w)
    dy, mean, rstd = K.layernorm_fwd(D.from_numpy(x), D.from_numpy(w), D.from_numpy(b))
    assert rel_err(dy.numpy(), y) <= TOL[dt]
    assert rel_err(rstd.numpy(), cache[1].reshape(-1)) <= TOL[dt]
    dx, dw, db = K.layernorm_bwd(D.from_numpy(g), D.from_numpy(x), D.from_numpy(w), mean, rstd)
    assert rel_err(dx.numpy(), gx) <= TOL[dt]
    assert rel_err(dw.numpy(), gw) <= TOL[dt]
    assert rel_err(db.numpy(), gb) <= TOL[dt]
    dx2, dw2, _ = K.layernorm_bwd(D.from_numpy(g), D.from_numpy(x), D.from_numpy(w), mean, rstd)
    assert bits_equal(dx2.numpy(), dx.numpy()) and bits_equal(dw2.numpy(), dw.numpy())


@pytest.mark.parametrize("dt", [np.float64, np.float32])
@pytest.mark.parametrize("shape", [(4096, 768), (33, 1000), (3, 17), (9, 5000)])
def test_layernorm_backward_with_addend_bits(dev, dt, shape):
    """dtmi_layernorm_bwd_add: dx = addend + the input gradient in the same
    pass, bit for bit the separate sum addend + dx (the backward engine's
    order); dgamma and dbeta unchanged."""
    D, K = _dev()
    rng = np.random.default_rng(shape[0] + shape[1])
    C = shape[-1]
    x = D.from_numpy(rng.standard_normal(shape).astype(dt))
    w = D.from_numpy((1 + 0.01 * rng.standard_normal(C)).astype(dt))
    b = D.from_numpy((0.01 * rng.standard_normal(C)).astype(dt))
    g = D.from_numpy(rng.standard_normal(shape).astype(dt))
    pend = D.from_numpy(rng.standard_normal(shape).astype(dt))
    _, mean, rstd = K.layernorm_fwd(x, w, b)
    dx, dw, db = K.layernorm_bwd(g, x, w, mean, rstd)
    dxa, dwa, dba = K.layernorm_bwd(g, x, w, mean, rstd, dx_addend=pend)
    assert bits_equal(dxa.numpy(), K.binary("add", pend, dx).numpy())
    assert bits_equal(dwa.numpy(), dw.numpy()) and bits_equal(dba.numpy(), db.numpy())


def test_layernorm_backward_rejects_an_addend_overlapping_dx(dev):
    """An addend that shares bytes with dx without being dx (a shifted view of
    one buffer) is refused before any launch; disjoint neighbours are fine."""
    import ctypes
    from dtmi import _lib
    D, K = _dev()
    rows, C = 8, 64
    x = D.from_numpy(np.random.default_rng(0).standard_normal((rows, C)).astype(np.float32))
    w, b = D.full((C,), 1.0, np.float32), D.zeros((C,), np.float32)
    g = D.full((rows, C), 0.5, np.float32)
    _, mean, rstd = K.layernorm_fwd(x, w, b)
    buf = D.zeros((3 * rows * C,), np.float32)
    dw, db = D.empty((C,), np.float32), D.empty((C,), np.float32)

    def call(dx_off, add_off):
        return _lib.lib().dtmi_layernorm_bwd_add(
            _lib.F32, ctypes.c_void_p(buf.ptr + 4 * dx_off), dw.ptr, db.ptr, g.ptr, x.ptr, w.ptr, mean.ptr, rstd.ptr,
            ctypes.c_void_p(buf.ptr + 4 * add_off), rows, C, 0)
    for dx_off, add_off in ((0, 1), (C, 0), (0, rows * C - 1), (0, 0)):
        assert call(dx_off, add_off) == 1, (dx_off, add_off)  # DTMI_ERR_INVALID
    assert call(0, rows * C) == 0 and call(2 * rows * C, rows * C) == 0
    _lib.sync()


def test_layernorm_backward_parts_rejects_overlaps_and_part_counts(dev):
    """dtmi_layernorm_bwd_parts refuses, before any launch, partials or an
    addend that share bytes with dx and part counts outside 1..64; disjoint
    neighbours in one buffer are fine."""
    import ctypes
    from dtmi import _lib
    D, K = _dev()
    rows, C, n = 8, 64, 2
    x = D.from_numpy(np.random.default_rng(1).standard_normal((rows, C)).astype(np.float32))
    w, b = D.full((C,), 1.0, np.float32), D.zeros((C,), np.float32)
    _, mean, rstd = K.layernorm_fwd(x, w, b)
    e = rows * C
    buf = D.full((5 * e,), 0.25, np.float32)
    dw, db = D.empty((C,), np.float32), D.empty((C,), np.float32)

    def call(dx_off, parts_off, nparts=n, add_off=None):
        add = ctypes.c_void_p(buf.ptr + 4 * add_off) if add_off is not None else None
        return _lib.lib().dtmi_layernorm_bwd_parts(
            _lib.F32, ctypes.c_void_p(buf.ptr + 4 * dx_off), dw.ptr, db.ptr, ctypes.c_void_p(buf.ptr + 4 * parts_off),
            nparts, x.ptr, w.ptr, mean.ptr, rstd.ptr, add, rows, C, 0)
    # dx inside the partials, straddling their end, or at their start
    for dx_off, parts_off in ((e, 0), (2 * e - 1, 0), (0, 0), (e, 1)):
        assert call(dx_off, parts_off) == 1, (dx_off, parts_off)  # DTMI_ERR_INVALID
    assert call(4 * e, 0, add_off=4 * e + 3) == 1  # addend overlapping dx
    assert call(4 * e, 0, nparts=0) == 1 and call(4 * e, 0, nparts=65) == 1
    assert call(2 * e, 0) == 0 and call(0, e) == 0 and call(4 * e, 0, add_off=2 * e) == 0
    _lib.sync()


@pytest.mark.parametrize("shape", [(40, 3000), (1100, 4096)])
def test_layernorm_long_float32_rows(dev, shape):
    """float32 rows of 12 and 16 vectors per lane: the backward loads each
    vector where it is used instead of prefetching the next row."""
    test_layernorm_forward_backward(dev, np.float32, shape)


@pytest.mark.parametrize("dt", [np.float64, np.float32])
@pytest.mark.parametrize("rows,V", [(6, 5), (256, 65), (64, 50304), (33, 1003)])
def test_cross_entropy_forward_backward(dev, dt, rows, V):
    D, K = _dev()
    rng = np.random.default_rng(rows + V)
    z = (rng.standard_normal((rows, V)) * 3).astype(dt)
    t = rng.integers(0, V, rows)
    loss, cache = ops.cross_entropy_fwd(z, t)
    gscale = np.asarray(0.25, dtype=dt)  # the `loss * (1/n_micro)` upstream gradient
    gz = ops.cross_entropy_bwd(gscale, z, t, cache)
    dz = D.from_numpy(z)
    dtgt = D.from_numpy(t.astype(np.int64))
    dloss, rmax, rsum = K.xent_fwd(dz, dtgt)
    assert rel_err(dloss.numpy(), loss) <= TOL[dt]
    ggrad = K.xent_bwd(dz, dtgt, rmax, rsum, g=D.from_numpy(gscale.reshape(1)))
    assert rel_err(ggrad.numpy(), gz) <= TOL[dt]


@pytest.mark.parametrize("dt", [np.float32, np.float64])
@pytest.mark.parametrize("rows,V", [(64, 50304), (8, 65536), (16, 4), (33, 1003), (8, 65540), (256, 65)])
def test_cross_entropy_single_pass_forward_and_gradient(dev, dt, rows, V):
    """dtmi_xent_fused (one read of the logits for float32 rows of up to 65536,
    the two-kernel form otherwise) against the oracle, then the in-place
    rescale for upstream gradients 1 (no change) and 0.25."""
    D, K = _dev()
    rng = np.random.default_rng(rows * 3 + V)
    z = (rng.standard_normal((rows, V)) * 3).astype(dt)
    t = rng.integers(0, V, rows)
    loss, cache = ops.cross_entropy_fwd(z, t)
    dz, dtgt = D.from_numpy(z), D.from_numpy(t.astype(np.int64))
    dloss, rmax, rsum, dl = K.xent_fused(dz, dtgt)
    assert rel_err(dloss.numpy(), loss) <= TOL[dt]
    g1 = ops.cross_entropy_bwd(np.asarray(1.0, dtype=dt), z, t, cache)
    assert rel_err(dl.numpy(), g1) <= TOL[dt]
    before = dl.numpy()
    K.xent_grad_scale(dl, D.from_numpy(np.ones(1, dt)))
    assert bits_equal(dl.numpy(), before)
    gq = ops.cross_entropy_bwd(np.asarray(0.25, dtype=dt), z, t, cache)
    K.xent_grad_scale(dl, D.from_numpy(np.full(1, 0.25, dt)))
    assert rel_err(dl.numpy(), gq) <= TOL[dt]
    # the saved row statistics serve the two-kernel backward as well
    assert rel_err(K.xent_bwd(dz, dtgt, rmax, rsum, g_host=1.0).numpy(), g1) <= TOL[dt]


@pytest.mark.parametrize("dt", [np.float64, np.float32])
def test_softmax_backward(dev, dt):
    D, K = _dev()
    rng = np.random.default_rng(7)
    s = rng.standard_normal((16 * 12 * 4, 256))
    p = (np.exp(s) / np.exp(s).sum(-1, keepdims=True)).astype(dt)
    dp = rng.standard_normal(p.shape).astype(dt)
    ref = ops.softmax_bwd(p, dp)
    assert rel_err(K.softmax_bwd(D.from_numpy(p), D.from_numpy(dp)).numpy(), ref) <= TOL[dt]


@pytest.mark.parametrize("dt", [np.float64, np.float32])
@pytest.mark.parametrize("V,C,shape", [(3, 4, (2, 3)), (65, 64, (8, 32)), (50304, 768, (8, 1024)), (32, 16, (8, 32))])
def test_embedding_forward_and_bit_exact_scatter_add(dev, dt, V, C, shape):
    D, K = _dev()
    rng = np.random.default_rng(V)
    w = rng.standard_normal((V, C)).astype(dt)
    idx = rng.integers(0, V, shape)
    if V == 3:
        idx = np.array([[0, 2, 2], [1, 0, 2]])  # dtrain tests/test_autograd.py:61-63
    g = rng.standard_normal(shape + (C,)).astype(dt)
    didx = D.from_numpy(idx.astype(np.int64).reshape(-1))
    out = K.embedding_fwd(D.from_numpy(w), didx, shape)
    assert bits_equal(out.numpy(), w[idx])
    segs = K.embedding_segments(didx)
    _check_segments(idx, segs)
    dw = K.embedding_bwd(D.from_numpy(g), V, segs)
    assert bits_equal(dw.numpy(), ops.embedding_bwd(g, (V, C), dt, idx))


def _check_segments(idx, segs):
    """The device sort equals NumPy's stable argsort; segment s covers the
    positions of row[s] in increasing order (np.add.at's order)."""
    flat = np.asarray(idx).reshape(-1)
    perm, start, row, nseg = (x.numpy() for x in segs)
    order = np.argsort(flat, kind="stable")
    rows = np.unique(flat)
    assert nseg[0] == rows.size
    assert np.array_equal(perm, order)
    assert np.array_equal(row[:rows.size], rows)
    first = np.flatnonzero(np.r_[True, flat[order][1:] != flat[order][:-1]])[:rows.size]
    assert np.array_equal(start[:rows.size + 1], np.r_[first, flat.size])


@pytest.mark.parametrize("n,V", [(0, 5), (1, 3), (8191, 50304), (8192, 7), (8193, 50304), (20000, 64),
                                 (65536, 50304), (100003, 1000)])
def test_embedding_segments_on_device(dev, n, V):
    """Chunk sorts of 8192 keys, merge passes (n above 8192, uneven last runs)
    and the segment scan across 1024-key blocks, against NumPy's stable
    argsort; then the table gradient bit-equal to np.add.at."""
    D, K = _dev()
    rng = np.random.default_rng(n + V)
    idx = rng.integers(0, V, n)
    segs = K.embedding_segments(D.from_numpy(idx.astype(np.int64)))
    _check_segments(idx, segs)
    if n:
        g = rng.standard_normal((n, 8)).astype(np.float32)
        dw = K.embedding_bwd(D.from_numpy(g), V, segs)
        assert bits_equal(dw.numpy(), ops.embedding_bwd(g, (V, 8), np.float32, idx))


def _gemm_ref(a, b, akc, bkc):
    A = a if akc else np.swapaxes(a, -1, -2)
    B = b if not bkc else np.swapaxes(b, -1, -2)
    return A @ B


@pytest.mark.parametrize("dt", [np.float64, np.float32])
@pytest.mark.parametrize("akc,bkc", [(True, False), (True, True), (False, False), (False, True)])
@pytest.mark.parametrize("M,N,K", [(256, 192, 64), (300, 65, 64), (1, 1, 1), (129, 257, 33), (8, 5, 7),
                                   (512, 2304, 768), (132, 68, 36), (260, 132, 1000), (4, 4, 4)])
def test_gemm_layouts_and_ragged_shapes(dev, dt, akc, bkc, M, N, K):
    D, K_ = _dev()
    rng = np.random.default_rng(M * 7 + N * 3 + K)
    a = rng.standard_normal((M, K) if akc else (K, M)).astype(dt)
    b = rng.standard_normal((N, K) if bkc else (K, N)).astype(dt)
    bias = rng.standard_normal(N).astype(dt)
    ref = _gemm_ref(a.astype(np.float64), b.astype(np.float64), akc, bkc) + bias
    got = K_.gemm(D.from_numpy(a), D.from_numpy(b), a_kcontig=akc, b_kcontig=bkc, bias=D.from_numpy(bias)).numpy()
    assert rel_err(got, ref) <= TOL[dt]


@pytest.mark.parametrize("dt", [np.float64, np.float32])
def test_gemm_split_k_is_deterministic_and_correct(dev, dt):
    D, K_ = _dev()
    rng = np.random.default_rng(11)
    a = rng.standard_normal((4096, 256)).astype(dt)  # X: [M=4096, K=256] -> dW = X^T dY
    g = rng.standard_normal((4096, 384)).astype(dt)
    ref = a.astype(np.float64).T @ g.astype(np.float64)
    outs = [K_.gemm(D.from_numpy(a), D.from_numpy(g), a_kcontig=False, b_kcontig=False, splits=s).numpy()
            for s in (1, 4, 4, 0)]
    for o in outs:
        assert rel_err(o, ref) <= TOL[dt]
    assert bits_equal(outs[1], outs[2])


@pytest.mark.parametrize("dt", [np.float64, np.float32])
@pytest.mark.parametrize("akc,bkc", [(True, False), (False, False), (True, True)])
def test_gemm_split_k_with_partial_last_tile(dev, dt, akc, bkc):
    """K = 1000 over 3 splits: the last split ends in a partial k-tile."""
    D, K_ = _dev()
    rng = np.random.default_rng(13)
    M, N, K = 200, 132, 1000
    a = rng.standard_normal((M, K) if akc else (K, M)).astype(dt)
    b = rng.standard_normal((N, K) if bkc else (K, N)).astype(dt)
    ref = _gemm_ref(a.astype(np.float64), b.astype(np.float64), akc, bkc)
    outs = [K_.gemm(D.from_numpy(a), D.from_numpy(b), a_kcontig=akc, b_kcontig=bkc, splits=s).numpy()
            for s in (1, 3, 3)]
    for o in outs:
        assert rel_err(o, ref) <= TOL[dt]
    assert bits_equal(outs[1], outs[2])


@pytest.mark.parametrize("dt", [np.float64, np.float32])
@pytest.mark.parametrize("akc,bkc", [(True, False), (True, True), (False, False), (False, True)])
def test_gemm_direct_lds_kernel_matches_register_staged_kernel_bitwise(dev, dt, akc, bkc):
    """16-byte aligned operands take the direct-to-LDS kernel; the same values
    one element off alignment take the register-staged kernel. Both feed the
    MFMAs the same k order, so the products agree to the bit (128 x 128
    block tiles, one split, ragged M and N, a partial last k-tile)."""
    D, K_ = _dev()
    rng = np.random.default_rng(41)
    M, N, K = 300, 260, 1000
    a = rng.standard_normal((M, K) if akc else (K, M)).astype(dt)
    b = rng.standard_normal((N, K) if bkc else (K, N)).astype(dt)
    bias = D.from_numpy(rng.standard_normal(N).astype(dt))
    db = D.from_numpy(b)
    big = D.empty((a.size + 1,), dt)
    a_off = big[1:1 + a.size].reshape(*a.shape)
    a_off.assign(a)
    assert a_off.ptr % 16 != 0
    aligned_ = K_.gemm(D.from_numpy(a), db, a_kcontig=akc, b_kcontig=bkc, bias=bias, splits=1).numpy()
    staged = K_.gemm(a_off, db, a_kcontig=akc, b_kcontig=bkc, bias=bias, splits=1).numpy()
    ref = _gemm_ref(a.astype(np.float64), b.astype(np.float64), akc, bkc) + bias.numpy()
    assert rel_err(aligned_, ref) <= TOL[dt]
    assert bits_equal(aligned_, staged)


@pytest.mark.parametrize("dt", [np.float64, np.float32])
@pytest.mark.parametrize("akc,bkc", [(True, False), (False, True)])
def test_batched_gemm_direct_lds_kernel_matches_register_staged_kernel_bitwise(dev, dt, akc, bkc):
    """Batched products (batch strides of whole matrices, as the attention's
    wide path uses them): the direct-to-LDS kernel on aligned operands and the
    register-staged kernel on the same values off alignment give the same
    bits, split into K ranges or not."""
    D, K_ = _dev()
    rng = np.random.default_rng(43)
    Bt, M, N, K = 3, 136, 200, 520
    a = rng.standard_normal((Bt, M, K) if akc else (Bt, K, M)).astype(dt)
    b = rng.standard_normal((Bt, N, K) if bkc else (Bt, K, N)).astype(dt)
    db = D.from_numpy(b)
    big = D.empty((a.size + 1,), dt)
    a_off = big[1:1 + a.size].reshape(*a.shape)
    a_off.assign(a)
    ref = _gemm_ref(a.astype(np.float64), b.astype(np.float64), akc, bkc)
    for splits in (1, 2):
        aligned_ = K_.gemm(D.from_numpy(a), db, a_kcontig=akc, b_kcontig=bkc, splits=splits).numpy()
        staged = K_.gemm(a_off, db, a_kcontig=akc, b_kcontig=bkc, splits=splits).numpy()
        assert rel_err(aligned_, ref) <= TOL[dt]
        assert bits_equal(aligned_, staged)


@pytest.mark.parametrize("akc,bkc", [(True, False), (True, True), (False, False), (False, True)])
def test_gemm_large_tile_ragged_edges_and_k_tail(dev, akc, bkc):
    """float32 shapes whose k range per block is long enough for the 256 x 128
    block tile: M, N not multiples of the tile, K = 2052 over 2 splits (the
    second ends in a partial k-tile); split results bit-identical run to run."""
    D, K_ = _dev()
    rng = np.random.default_rng(21)
    M, N, K = 2000, 2040, 2052
    a = rng.standard_normal((M, K) if akc else (K, M)).astype(np.float32)
    b = rng.standard_normal((N, K) if bkc else (K, N)).astype(np.float32)
    ref = _gemm_ref(a.astype(np.float64), b.astype(np.float64), akc, bkc)
    da, db = D.from_numpy(a), D.from_numpy(b)
    outs = [K_.gemm(da, db, a_kcontig=akc, b_kcontig=bkc, splits=s).numpy() for s in (0, 0, 1)]
    for o in outs:
        assert rel_err(o, ref) <= TOL[np.float32]
    assert bits_equal(outs[0], outs[1])


@pytest.mark.parametrize("akc,bkc,which", [(True, False, "A"), (False, False, "A"), (True, False, "B"),
                                           (True, True, "B")])
def test_gemm_operand_crossing_a_4gib_address_boundary(dev, akc, bkc, which):
    """float32 operands placed so that the per-k-tile advance of the loads'
    64-bit base address carries into its high dword (a 4 GiB boundary is
    crossed inside the k loop); the result must match the reference."""
    D, K_ = _dev()
    M, N, K = 512, 384, 2048
    rng = np.random.default_rng(31)
    a = rng.standard_normal((M, K) if akc else (K, M)).astype(np.float32)
    b = rng.standard_normal((N, K) if bkc else (K, N)).astype(np.float32)
    big = D.empty(((4 << 30) // 4 + (64 << 20) // 4,), np.float32)
    boundary = -(-big.ptr // (1 << 32)) * (1 << 32)
    assert boundary + (32 << 20) <= big.ptr + big.nbytes
    # the operand starts a few k-tiles (or k-rows) before the boundary
    x = a if which == "A" else b
    lead = 5 * 64 if (akc if which == "A" else bkc) else 3 * 64 * x.shape[1]
    e0 = (boundary - big.ptr - lead) // 4
    view = big[e0:e0 + x.size].reshape(*x.shape)
    view.assign(x)
    other = D.from_numpy(b if which == "A" else a)
    da, db = (view, other) if which == "A" else (other, view)
    ref = _gemm_ref(a.astype(np.float64), b.astype(np.float64), akc, bkc)
    for splits in (1, 0):
        got = K_.gemm(da, db, a_kcontig=akc, b_kcontig=bkc, splits=splits).numpy()
        assert rel_err(got, ref) <= TOL[np.float32]


@pytest.mark.parametrize("dt", [np.float64, np.float32])
def test_batched_gemm(dev, dt):
    D, K_ = _dev()
    rng = np.random.default_rng(12)
    a = rng.standard_normal((3, 40, 24)).astype(dt)
    b = rng.standard_normal((3, 24, 56)).astype(dt)
    got = K_.gemm(D.from_numpy(a), D.from_numpy(b)).numpy()
    assert rel_err(got, a @ b) <= TOL[dt]


@pytest.mark.parametrize("dt", [np.float64, np.float32])
def test_linear_forward_backward_at_layernorm_linear_workload(dev, dt):
    """The LayerNorm + Linear backward workload: x [16384, 768], W [768, 3072],
    y = LN(x) W + b; dX, dW, db, dgamma, dbeta against the oracle."""
    D, K = _dev()
    rng = np.random.default_rng(2)
    M, Cin, N = 16384, 768, 3072
    x = rng.standard_normal((M, Cin)).astype(dt)
    W = (rng.standard_normal((Cin, N)) * 0.02).astype(dt)
    b = np.zeros(N, dt)
    gamma = (1 + rng.standard_normal(Cin) * 0.01).astype(dt)
    beta = (rng.standard_normal(Cin) * 0.01).astype(dt)
    dY = rng.standard_normal((M, N)).astype(dt)
    h, cache = ops.layer_norm_fwd(x, gamma, beta)
    gh, gW = ops.matmul_bwd(dY, h, W)
    gb = ops.unbroadcast(dY, (N,))
    gx, ggam, gbet = ops.layer_norm_bwd(gh, cache, gamma)
    dx_, dW_, db_ = D.from_numpy(x), D.from_numpy(W), D.from_numpy(b)
    hd, mean, rstd = K.layernorm_fwd(dx_, D.from_numpy(gamma), D.from_numpy(beta))
    y = K.linear_fwd(hd, dW_, db_)
    assert rel_err(y.numpy(), h @ W + b) <= TOL[dt]
    dh, dW, db = K.linear_bwd(hd, dW_, D.from_numpy(dY))
    assert rel_err(dh.numpy(), gh) <= TOL[dt]
    assert rel_err(dW.numpy(), gW) <= TOL[dt]
    assert rel_err(db.numpy(), gb) <= TOL[dt]
    dx, dgam, dbet = K.layernorm_bwd(dh, dx_, D.from_numpy(gamma), mean, rstd)
    assert rel_err(dx.numpy(), gx) <= TOL[dt]
    assert rel_err(dgam.numpy(), ggam) <= TOL[dt]
    assert rel_err(dbet.numpy(), gbet) <= TOL[dt]


@pytest.mark.parametrize("dt", [np.float64, np.float32])
@pytest.mark.parametrize("K,N,parts,n", [(768, 2304, 2, 2), (768, 2304, 4, 2), (768, 3072, 2, 2),
                                         (768, 3072, 4, 2), (768, 50304, 4, 4)])
def test_layernorm_backward_adds_the_split_k_partials_of_dy(dev, dt, K, N, parts, n):
    """The qkv / fc / vocabulary-head input gradient ([8192, 768] = dY W^T
    over N = 2304, 3072 or 50304) left as split-K partials (at most `parts`;
    the float32 products split into n: two, or four for the head) and summed
    inside the LayerNorm backward: the same bits as summing first
    (dtmi_linear_bwd_dx) and then dtmi_layernorm_bwd, with and without the
    residual addend; and the partials' value equal to the summed product."""
    D, K_ = _dev()
    rng = np.random.default_rng(K + N)
    M = 8192
    x = D.from_numpy(rng.standard_normal((M, K)).astype(dt))
    lw = D.from_numpy((1 + 0.01 * rng.standard_normal(K)).astype(dt))
    lb = D.from_numpy((0.01 * rng.standard_normal(K)).astype(dt))
    W = D.from_numpy((rng.standard_normal((K, N)) * 0.02).astype(dt))
    dY = D.from_numpy(rng.standard_normal((M, N)).astype(dt))
    pend = D.from_numpy(rng.standard_normal((M, K)).astype(dt))
    h, mean, rstd = K_.layernorm_fwd(x, lw, lb)
    dh, _, _ = K_.linear_bwd(h, W, dY, need_db=False)
    dsplit, _, _ = K_.linear_bwd(h, W, dY, need_db=False, dx_parts=parts)
    if dt == np.float32:
        assert isinstance(dsplit, K_.SplitSum) and dsplit.n == n
    val = dsplit.value() if isinstance(dsplit, K_.SplitSum) else dsplit
    assert bits_equal(val.numpy(), dh.numpy())
    for addend in (None, pend):
        ref = K_.layernorm_bwd(dh, x, lw, mean, rstd, dx_addend=addend)
        got = K_.layernorm_bwd(dsplit, x, lw, mean, rstd, dx_addend=addend)
        for r, g_ in zip(ref, got):
            assert bits_equal(g_.numpy(), r.numpy())


@pytest.mark.parametrize("dt", [np.float64, np.float32])
@pytest.mark.parametrize("rows,C,n", [(4096, 768, 3), (33, 1000, 2), (9, 5000, 2), (64, 768, 4)])
def test_layernorm_backward_partials_outside_the_fused_load(dev, dt, rows, C, n):
    """dtmi_layernorm_bwd_parts where the partials are summed by a pass of
    their own first (more than two parts, unaligned rows, rows longer than 8
    vectors per lane): the bits of summing in order and dtmi_layernorm_bwd."""
    D, K_ = _dev()
    rng = np.random.default_rng(rows + C + n)
    x = D.from_numpy(rng.standard_normal((rows, C)).astype(dt))
    lw = D.from_numpy((1 + 0.01 * rng.standard_normal(C)).astype(dt))
    lb = D.from_numpy((0.01 * rng.standard_normal(C)).astype(dt))
    parts = D.from_numpy(rng.standard_normal((n, rows, C)).astype(dt))
    _, mean, rstd = K_.layernorm_fwd(x, lw, lb)
    s = K_.SplitSum(parts, n, (rows, C))
    ref = K_.layernorm_bwd(s.value(), x, lw, mean, rstd)
    got = K_.layernorm_bwd(s, x, lw, mean, rstd)
    for r, g_ in zip(ref, got):
        assert bits_equal(g_.numpy(), r.numpy())


@pytest.mark.parametrize("dt", [np.float64, np.float32])
@pytest.mark.parametrize("M,K,N", [(1024, 256, 512), (256, 4096, 96), (300, 68, 132), (2048, 2048, 2048),
                                   (4096, 1024, 2048)])
def test_fused_linear_epilogues_equal_the_unfused_ops(dev, dt, M, K, N):
    """Residual add, GELU and GELU backward in the GEMM epilogue give the same
    bits as the separate kernels (with and without split-K)."""
    D, K_ = _dev()
    rng = np.random.default_rng(M + K + N)
    x = D.from_numpy(rng.standard_normal((M, K)).astype(dt))
    w = D.from_numpy((rng.standard_normal((K, N)) * 0.05).astype(dt))
    b = D.from_numpy(rng.standard_normal(N).astype(dt))
    r = D.from_numpy(rng.standard_normal((M, N)).astype(dt))
    y0 = K_.linear_fwd(x, w, b)
    y_res, none = K_.linear_fwd_fused(x, w, b, residual=r)
    assert none is None
    assert bits_equal(y_res.numpy(), K_.binary("add", r, y0).numpy())
    h, act = K_.linear_fwd_fused(x, w, b, gelu=True)
    assert bits_equal(h.numpy(), y0.numpy())
    assert bits_equal(act.numpy(), K_.gelu_fwd(y0).numpy())
    # backward through gelu: dx of the pre-activation whose GELU is the input x
    pre = D.from_numpy(rng.standard_normal((M, K)).astype(dt))
    g = D.from_numpy(rng.standard_normal((M, N)).astype(dt))
    dx_plain, _, _ = K_.linear_bwd(x, w, g, need_db=False)
    dx_fused, _, _ = K_.linear_bwd(x, w, g, need_db=False, gelu_pre=pre)
    assert bits_equal(dx_fused.numpy(), K_.gelu_bwd(pre, dx_plain).numpy())
    ref = (x.numpy().astype(np.float64) @ w.numpy().astype(np.float64)) + b.numpy() + r.numpy()
    assert rel_err(y_res.numpy(), ref) <= TOL[dt]


@pytest.mark.parametrize("dt", [np.float32, np.float64])
@pytest.mark.parametrize("M,K,N,resid", [(8192, 768, 768, True), (8192, 3072, 768, True), (512, 3072, 768, False),
                                         (300, 64, 2304, True), (96, 200, 130, True)])
def test_linear_with_the_next_layernorm_equals_the_separate_ops(dev, dt, M, K, N, resid):
    """dtmi_linear_fwd_ln: y = residual + (x @ w + b) and h = layer_norm(y) in
    one call (split-K sum, bias, residual and LayerNorm in one row pass when
    the product is split over K) -- bit for bit the separate fused Linear and
    LayerNorm kernels, on split and unsplit shapes, ragged rows and float64."""
    D, K_ = _dev()
    rng = np.random.default_rng(M + K + N)
    x = D.from_numpy(rng.standard_normal((M, K)).astype(dt))
    w = D.from_numpy((rng.standard_normal((K, N)) * 0.02).astype(dt))
    b = D.from_numpy((rng.standard_normal(N) * 0.1).astype(dt))
    r = D.from_numpy(rng.standard_normal((M, N)).astype(dt)) if resid else None
    lw = D.from_numpy((1 + 0.1 * rng.standard_normal(N)).astype(dt))
    lb = D.from_numpy((0.1 * rng.standard_normal(N)).astype(dt))
    y, h, mean, rstd = K_.linear_fwd_ln(x, w, b, r, lw, lb)
    y2, _ = K_.linear_fwd_fused(x, w, b, residual=r)
    h2, mean2, rstd2 = K_.layernorm_fwd(y2, lw, lb)
    for a, ref in ((y, y2), (h, h2), (mean, mean2), (rstd, rstd2)):
        assert bits_equal(a.numpy(), ref.numpy())
    # and the values: the oracle's Linear + residual and LayerNorm
    ref_y = x.numpy() @ w.numpy() + b.numpy() + (r.numpy() if resid else 0)
    assert rel_err(y.numpy(), ref_y) <= (1e-5 if dt == np.float32 else 1e-12)
    ref_h, _ = ops.layer_norm_fwd(ref_y, lw.numpy(), lb.numpy())
    assert rel_err(h.numpy(), ref_h) <= (1e-5 if dt == np.float32 else 1e-12)
