"""Causal attention (flash-style forward + recompute backward, MFMA) on the GPU
against the oracle restatement of dtrain's causal_attention.

Bar: float64 normwise relative error <= 1e-12; float32 <= 1e-5 (dtrain itself
computes the float32 case in float64 under NumPy 2; the oracle reproduces that).
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


def _check(D, K, q, k, v, g, dt):
    o_ref, p, scale = ops.attention_fwd(q, k, v)
    gq, gk, gv = ops.attention_bwd(g, q, k, v, p, scale)
    m_ref, l_ref = ops.row_stats(q, k)
    dq_, dk_, dv_ = D.from_numpy(q), D.from_numpy(k), D.from_numpy(v)
    o, rmax, rsum = K.attn_fwd(dq_, dk_, dv_)
    assert rel_err(o.numpy(), o_ref) <= TOL[dt]
    # the kernels keep the row max in base-2 units (log2(e) * max), for exp2
    assert rel_err(rmax.numpy(), m_ref * np.log2(np.e)) <= TOL[dt]
    assert rel_err(rsum.numpy(), l_ref) <= TOL[dt]
    gq_d, gk_d, gv_d = K.attn_bwd(dq_, dk_, dv_, o, D.from_numpy(g), rmax, rsum)
    assert rel_err(gq_d.numpy(), gq) <= TOL[dt]
    assert rel_err(gk_d.numpy(), gk) <= TOL[dt]
    assert rel_err(gv_d.numpy(), gv) <= TOL[dt]


@pytest.mark.parametrize("dt", [np.float64, np.float32])
@pytest.mark.parametrize("shape", [(1, 2, 4, 3), (1, 2, 8, 4), (2, 2, 5, 4), (8, 4, 32, 16), (2, 3, 100, 64),
                                   (1, 1, 257, 33), (16, 12, 256, 64), (2, 3, 32, 64), (1, 2, 64, 64),
                                   (2, 2, 96, 64)])
def test_attention_forward_backward(dev, dt, shape):
    D, K = _dev()
    rng = np.random.default_rng(sum(shape))
    q, k, v, g = (rng.standard_normal(shape).astype(dt) for _ in range(4))
    _check(D, K, q, k, v, g, dt)


@pytest.mark.parametrize("shape", [(1, 2, 16, 64), (2, 3, 208, 64), (3, 2, 512, 64), (1, 2, 2048, 64)])
def test_float64_backward_at_head_dim_64(dev, shape):
    """float64, D = 64 on the aligned path (64-key blocks of 16 per wave, dS
    stored at wave-uniform row offsets and read back through a buffer
    resource by the dQ pass; one tile, T not a multiple of 32 or of 64, and
    T 2048, where a (batch, head)'s dS spans 32 MB), against the oracle at
    1e-12."""
    D, K = _dev()
    rng = np.random.default_rng(sum(shape) + 64)
    q, k, v, g = (rng.standard_normal(shape) for _ in range(4))
    _check(D, K, q, k, v, g, np.float64)


@pytest.mark.parametrize("T", [512, 640, 768, 896, 1024, 2048])
def test_forward_over_many_key_tiles(dev, T):
    """T of 512 to 2048 on the aligned float32 path (the paired-range
    forward, 33 to 129 key tiles of 16 per query tile pair), where the forward's
    reference max moves only when a score exceeds it by 2^8: oracle parity of
    the output, of the row statistics (the true max) and of the backward that
    reads them; identical bits over repeated calls."""
    D, K = _dev()
    rng = np.random.default_rng(T)
    q, k, v, g = (rng.standard_normal((2, 3, T, 64)).astype(np.float32) for _ in range(4))
    _check(D, K, q, k, v, g, np.float32)
    dq_, dk_, dv_ = D.from_numpy(q), D.from_numpy(k), D.from_numpy(v)
    runs = [tuple(x.numpy() for x in K.attn_fwd(dq_, dk_, dv_)) for _ in range(3)]
    for r in runs[1:]:
        for x, y in zip(runs[0], r):
            assert bits_equal(x, y)


@pytest.mark.parametrize("T", [4096, 8192])
def test_float32_attention_at_long_sequences(dev, T):
    """The float32 kernels accumulate in float32 where dtrain (NumPy 2)
    promotes to float64: at T = 4096 and 8192 (one batch element and head, so
    the oracle's T x T arrays stay within a few GB) the outputs, the row
    statistics and dQ, dK, dV stay within 1e-5 of the float64-promoted
    oracle."""
    D, K = _dev()
    rng = np.random.default_rng(T + 1)
    q, k, v, g = (rng.standard_normal((1, 1, T, 64)).astype(np.float32) for _ in range(4))
    _check(D, K, q, k, v, g, np.float32)


@pytest.mark.parametrize("T", [32, 64, 96, 160, 288, 352])
def test_backward_paired_ranges_at_every_pair_count(dev, T):
    """The float32 paired-range backward (16 x 16 tiles, key tile j with its
    mirror, dQ-pass blocks of query-tile pairs) at T / 32 = 1, 2, 3, 5,
    9 and 11 pairs: blocks whose last waves have no pair, one and two key
    tiles per dQ step, a single pair; dQ, dK and dV against the oracle, and
    identical bits over repeated calls."""
    D, K = _dev()
    rng = np.random.default_rng(T + 7)
    q, k, v, g = (rng.standard_normal((2, 3, T, 64)).astype(np.float32) for _ in range(4))
    _check(D, K, q, k, v, g, np.float32)
    dq_, dk_, dv_, dg_ = D.from_numpy(q), D.from_numpy(k), D.from_numpy(v), D.from_numpy(g)
    o, rmax, rsum = K.attn_fwd(dq_, dk_, dv_)
    runs = [tuple(x.numpy() for x in K.attn_bwd(dq_, dk_, dv_, o, dg_, rmax, rsum)) for _ in range(3)]
    for r in runs[1:]:
        for x, y in zip(runs[0], r):
            assert bits_equal(x, y)


@pytest.mark.parametrize("B,H,T", [(40, 8, 256), (36, 4, 352), (40, 8, 512)])
def test_paired_grid_shapes_agree_bit_for_bit(dev, B, H, T):
    """The float32 paired-range passes pick their grids by size: the dQ pass
    takes four query-tile pairs per block when there are at least two such
    blocks per CU, else two pairs with each query tile's d-tiles split over two
    waves; the key pass and the forward take several tile pairs per block when
    one pair per block would need more than one round of resident blocks (at
    T 352 the key pass's 11 pairs do not divide evenly over the blocks; at
    T 512 the forward takes two pairs per block). Each order of additions is
    the same either way, so a (batch, head) gets the same bits: the full batch
    against its first two batch elements alone (split d-tiles, one pair per
    block), and those against the oracle."""
    D, K = _dev()
    rng = np.random.default_rng(B + T)
    q, k, v, g = (rng.standard_normal((B, H, T, 64)).astype(np.float32) for _ in range(4))

    def bwd(sl):
        x = [D.from_numpy(np.ascontiguousarray(t[sl])) for t in (q, k, v, g)]
        o, rmax, rsum = K.attn_fwd(x[0], x[1], x[2])
        return [t.numpy() for t in K.attn_bwd(x[0], x[1], x[2], o, x[3], rmax, rsum) + (o, rmax, rsum)]
    full, part = bwd(slice(0, B)), bwd(slice(0, 2))
    assert bits_equal(full[3][:2], part[3])  # the forward's output
    assert bits_equal(full[4][:2], part[4]) and bits_equal(full[5][:2], part[5])  # its row statistics
    full, part = full[:3], part[:3]
    for a, b in zip(full, part):
        assert bits_equal(a[:2], b)
    o_ref, p, scale = ops.attention_fwd(q[:2], k[:2], v[:2])
    for a, ref in zip(part, ops.attention_bwd(g[:2], q[:2], k[:2], v[:2], p, scale)):
        assert rel_err(a, ref) <= TOL[np.float32]


@pytest.mark.parametrize("dt", [np.float32, np.float64])
def test_attention_golden_from_dtrain(dev, golden, dt):
    D, K = _dev()
    G = golden("dtrain_attention.npz")
    key = np.dtype(dt).name
    q, k, v, g = (G[f"{key}/{s}"] for s in "qkvg")
    o, rmax, rsum = K.attn_fwd(D.from_numpy(q), D.from_numpy(k), D.from_numpy(v))
    assert rel_err(o.numpy(), G[f"{key}/o"]) <= TOL[dt]
    gq, gk, gv = K.attn_bwd(D.from_numpy(q), D.from_numpy(k), D.from_numpy(v), o, D.from_numpy(g), rmax, rsum)
    assert rel_err(gq.numpy(), G[f"{key}/gq"]) <= TOL[dt]
    assert rel_err(gk.numpy(), G[f"{key}/gk"]) <= TOL[dt]
    assert rel_err(gv.numpy(), G[f"{key}/gv"]) <= TOL[dt]


@pytest.mark.parametrize("dt", [np.float32, np.float64])
def test_attention_on_fused_qkv_layout(dev, dt):
    """q, k, v as strided views of a [B, T, 3, H, D] projection output (the
    reshape/transpose/split of dtrain/nn.py:100-103), outputs written into
    [B, T, H, D] and [B, T, 3, H, D] buffers."""
    D, K = _dev()
    B, T, H, Dh = 2, 96, 3, 16
    rng = np.random.default_rng(4)
    qkv = rng.standard_normal((B, T, 3, H, Dh)).astype(dt)
    g = rng.standard_normal((B, T, H, Dh)).astype(dt)
    q, k, v = (np.ascontiguousarray(qkv[:, :, i].transpose(0, 2, 1, 3)) for i in range(3))
    gh = np.ascontiguousarray(g.transpose(0, 2, 1, 3))
    o_ref, p, scale = ops.attention_fwd(q, k, v)
    gq, gk, gv = ops.attention_bwd(gh, q, k, v, p, scale)

    dqkv = D.from_numpy(qkv)
    t5 = dqkv.transpose(2, 0, 3, 1, 4)  # [3, B, H, T, D] view
    qd, kd, vd = t5[0], t5[1], t5[2]
    assert not qd.is_contiguous
    obuf = D.empty((B, T, H, Dh), dt)
    o, rmax, rsum = K.attn_fwd(qd, kd, vd, out=obuf.transpose(0, 2, 1, 3))
    assert rel_err(obuf.numpy().transpose(0, 2, 1, 3), o_ref) <= TOL[dt]
    gbuf = D.from_numpy(g)
    dbuf = D.full((B, T, 3, H, Dh), 7.0, dt)
    d5 = dbuf.transpose(2, 0, 3, 1, 4)
    K.attn_bwd(qd, kd, vd, obuf.transpose(0, 2, 1, 3), gbuf.transpose(0, 2, 1, 3), rmax, rsum,
               dq=d5[0], dk=d5[1], dv=d5[2])
    got = dbuf.numpy()
    assert rel_err(got[:, :, 0].transpose(0, 2, 1, 3), gq) <= TOL[dt]
    assert rel_err(got[:, :, 1].transpose(0, 2, 1, 3), gk) <= TOL[dt]
    assert rel_err(got[:, :, 2].transpose(0, 2, 1, 3), gv) <= TOL[dt]


@pytest.mark.parametrize("dt", [np.float64, np.float32])
@pytest.mark.parametrize("shape", [(1, 2, 4, 3), (2, 2, 5, 4), (2, 3, 100, 64), (1, 1, 257, 33), (16, 12, 256, 64),
                                   (1, 2, 384, 64)])
def test_recompute_dq_path_matches_oracle(dev, dt, shape):
    """With the dS workspace bound set to 0 the dQ pass recomputes S, P and
    dP from q, k, v, dO and the row statistics (the path taken above 4 GiB of
    dS): forward and backward against the oracle at the same bar."""
    D, K = _dev()
    rng = np.random.default_rng(sum(shape) + 7)
    q, k, v, g = (rng.standard_normal(shape).astype(dt) for _ in range(4))
    prev = K.attn_set_ds_limit(0)
    try:
        _check(D, K, q, k, v, g, dt)
    finally:
        K.attn_set_ds_limit(prev)
    assert prev == 4 << 30


def test_backward_without_the_ds_workspace_matches_with_it(dev):
    """B*H*T*T float32 above 4 GiB: the dQ pass recomputes dS instead of
    reading it from a workspace. Splitting the heads in two keeps each half
    under the limit (dS path); the two paths must agree to the float32 bar (their
    key passes add dK and dV over 6144 queries in different orders)."""
    D, K = _dev()
    B, H, T, Dh = 1, 32, 6144, 64
    rng = np.random.default_rng(21)
    hq, hk, hv, hg = (rng.standard_normal((B, H, T, Dh)).astype(np.float32) for _ in range(4))
    q, k, v, g = (D.from_numpy(x) for x in (hq, hk, hv, hg))
    o, rmax, rsum = K.attn_fwd(q, k, v)
    dq, dk, dv = K.attn_bwd(q, k, v, o, g, rmax, rsum)  # 4.8 GB of dS: recompute path
    ho, hm, hs = o.numpy(), rmax.numpy(), rsum.numpy()
    halves = []
    for lo in (0, H // 2):
        sl = slice(lo, lo + H // 2)
        sub = [D.from_numpy(np.ascontiguousarray(x[:, sl])) for x in (hq, hk, hv, ho, hg)]
        stats = [D.from_numpy(np.ascontiguousarray(x[:, sl])) for x in (hm, hs)]
        halves.append([t.numpy() for t in K.attn_bwd(*sub, *stats)])  # 2.4 GB each: dS path
    for i, full in enumerate((dq, dk, dv)):
        ref = np.concatenate([halves[0][i], halves[1][i]], axis=1)
        assert rel_err(full.numpy(), ref) <= 1e-5


@pytest.mark.parametrize("dt", [np.float64, np.float32])
@pytest.mark.parametrize("shape", [(2, 2, 64, 128), (1, 3, 100, 80), (2, 1, 33, 256)])
def test_head_dimensions_beyond_64(dev, dt, shape):
    """D > 64 (e.g. dtrain's --dim 256 --heads 2): scores materialised per batch
    element and the products as batched GEMMs; against the oracle."""
    D, K = _dev()
    rng = np.random.default_rng(sum(shape) + 1)
    q, k, v, g = (rng.standard_normal(shape).astype(dt) for _ in range(4))
    _check(D, K, q, k, v, g, dt)


@pytest.mark.parametrize("B,T,H,N", [(2, 64, 2, 96), (4, 1024, 12, 768)])
def test_rowsum_formed_by_the_projection_gradient(dev, B, T, H, N):
    """dtmi_linear_bwd_dx_rowdot (the projection that reads the attention
    output O: dO = dY W^T, plus rowsum(dO * O) per 64-wide head, in the split-K
    pass at the GPT-2-small shape and in a pass over dO at the small one) then
    dtmi_attn_bwd_rowsum: dO bit-equal to dtmi_linear_bwd_dx's, the row sums
    within float32 rounding of a float64 sum, and dq, dk, dv bit-equal to
    dtmi_attn_bwd computing the row sums itself (dtrain/autograd.py:242,
    nn.py:103-104)."""
    D, K = _dev()
    dt = np.float32
    C = H * 64
    rng = np.random.default_rng(B + T)
    qkv = rng.standard_normal((B, T, 3, H, 64)).astype(dt)
    w = (rng.standard_normal((C, N)) * 0.05).astype(dt)
    dy = rng.standard_normal((B * T, N)).astype(dt)
    dqkv = D.from_numpy(qkv)
    t5 = dqkv.transpose(2, 0, 3, 1, 4)
    obuf = D.empty((B, T, H, 64), dt)
    _, rmax, rsum = K.attn_fwd(t5[0], t5[1], t5[2], out=obuf.transpose(0, 2, 1, 3))
    x2 = obuf.reshape(B * T, C)
    dw_ = D.from_numpy(w)
    rs = D.empty((B * H * T,), dt)
    do_fused, _, _ = K.linear_bwd(x2, dw_, D.from_numpy(dy), need_db=False, rowdot=rs, rowdot_t=T)
    do_plain, _, _ = K.linear_bwd(x2, dw_, D.from_numpy(dy), need_db=False)
    assert np.array_equal(do_fused.numpy().view(np.uint32), do_plain.numpy().view(np.uint32))
    o64 = obuf.numpy().astype(np.float64).reshape(B, T, H, 64)
    g64 = do_plain.numpy().astype(np.float64).reshape(B, T, H, 64)
    ref = np.einsum("bthd,bthd->bht", o64, g64)
    assert rel_err(rs.numpy().reshape(B, H, T), ref) <= 1e-6
    g4 = do_plain.reshape(B, T, H, 64).transpose(0, 2, 1, 3)
    o4 = obuf.transpose(0, 2, 1, 3)
    a = [D.full((B, T, 3, H, 64), 3.0, dt) for _ in range(2)]
    for buf, drow in zip(a, (None, rs)):
        d5 = buf.transpose(2, 0, 3, 1, 4)
        K.attn_bwd(t5[0], t5[1], t5[2], o4, g4, rmax, rsum, dq=d5[0], dk=d5[1], dv=d5[2], drow=drow)
    assert np.array_equal(a[0].numpy().view(np.uint32), a[1].numpy().view(np.uint32))


@pytest.mark.parametrize("dt", [np.float64, np.float32])
@pytest.mark.parametrize("shape", [(2, 3, 256, 64), (1, 2, 128, 32)])
def test_results_written_through_unaligned_views(dev, dt, shape):
    """O, dQ, dK and dV written into views one element past a 16-byte
    boundary take the element-wise stores; aligned outputs take 16-byte
    stores. Both must give the same bits, and the values the oracle's."""
    D, K = _dev()
    rng = np.random.default_rng(sum(shape))
    hq, hk, hv, hg = (rng.standard_normal(shape).astype(dt) for _ in range(4))
    q, k, v, g = (D.from_numpy(x) for x in (hq, hk, hv, hg))
    n = int(np.prod(shape))

    def shifted():
        return D.empty((n + 1,), dt)[1:].reshape(*shape)

    o, rmax, rsum = K.attn_fwd(q, k, v)
    o2, rmax2, rsum2 = K.attn_fwd(q, k, v, out=shifted())
    assert o2.ptr % 16 != 0
    for a, b in ((o, o2), (rmax, rmax2), (rsum, rsum2)):
        assert bits_equal(a.numpy(), b.numpy())
    grads = K.attn_bwd(q, k, v, o, g, rmax, rsum)
    grads2 = K.attn_bwd(q, k, v, o, g, rmax, rsum, dq=shifted(), dk=shifted(), dv=shifted())
    for a, b in zip(grads, grads2):
        assert bits_equal(a.numpy(), b.numpy())
    o_ref, p, scale = ops.attention_fwd(hq, hk, hv)
    ref = ops.attention_bwd(hg, hq, hk, hv, p, scale)
    assert rel_err(o2.numpy(), o_ref) <= TOL[dt]
    for a, r in zip(grads2, ref):
        assert rel_err(a.numpy(), r) <= TOL[dt]
