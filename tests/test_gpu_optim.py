"""Optimizer / gradient-bucket kernels on the GPU against the oracle.

Bar: bit-exact for the fixed-order average and AdamW (float64 and float32,
built with -ffp-contract=off), bit-exact flatten, sum of squares within 1e-14
relative of dtrain's per-array float64 dot, identical bits across runs.
"""
import numpy as np
import pytest

from helpers import bits_equal, rel_err
from oracle import optim as O
from oracle.ddp import fixed_order_sum

pytestmark = pytest.mark.gpu


def _dev():
    from dtmi import device as D, kernels as K
    return D, K


def _adam_inputs(rng, n, dt):
    p = (rng.standard_normal(n) * 0.02).astype(dt)
    g = (rng.standard_normal(n) * 10.0 ** rng.uniform(-12, 1, n)).astype(dt)
    m = np.abs(rng.standard_normal(n) * 1e-4).astype(dt)
    v = np.abs(rng.standard_normal(n) * 1e-4).astype(dt)
    # edge values: exact zeros, subnormal-range and large gradients
    edge = np.array([0.0, -0.0, 1e-300 if dt == np.float64 else 1e-40, 1e30, -1e-30, 3.0, -7.5]).astype(dt)
    k = min(n, edge.size)
    g[:k] = edge[:k]
    v[:min(n, 3)] = 0
    return p, g, m, v


@pytest.mark.parametrize("dt", [np.float64, np.float32])
@pytest.mark.parametrize("n", [1, 3, 4097, 1_000_003])
@pytest.mark.parametrize("gscale", [1.0, 0.37109375123])
def test_adamw_flat_bit_exact(dev, dt, n, gscale):
    D, K = _dev()
    rng = np.random.default_rng(n)
    p, g, m, v = _adam_inputs(rng, n, dt)
    lr, b1, b2, eps, wd, t = 3e-4, 0.9, 0.95, 1e-8, 0.1, 101
    b1t, b2t = O.bias_corrections(b1, b2, t)
    dp, dg, dm, dv = (D.from_numpy(a) for a in (p, g, m, v))
    K.adamw(dp, dg, dm, dv, lr, b1, b2, eps, wd, b1t, b2t, gscale=gscale)
    gs = g * gscale  # dtrain/train.py:159 rounds the Python float to the array dtype
    O.adamw_update(p, gs, m, v, lr, b1, b2, eps, wd, b1t, b2t)
    assert bits_equal(dp.numpy(), p)
    assert bits_equal(dm.numpy(), m)
    assert bits_equal(dv.numpy(), v)


@pytest.mark.parametrize("dt", [np.float64, np.float32])
def test_adamw_misaligned_views_and_device_scale(dev, dt):
    """Views at odd element offsets take the scalar path; the clip factor comes
    from a device double."""
    D, K = _dev()
    rng = np.random.default_rng(5)
    n = 10_001
    p, g, m, v = _adam_inputs(rng, n + 1, dt)
    bufs = [D.from_numpy(a) for a in (p, g, m, v)]
    views = [b[1:] for b in bufs]
    s = 0.8123456789
    sdev = D.from_numpy(np.array([s]))
    b1t, b2t = O.bias_corrections(0.9, 0.95, 3)
    K.adamw(*views, 1e-3, 0.9, 0.95, 1e-8, 0.1, b1t, b2t, gscale=123.0, gscale_dev=sdev)
    pp, mm, vv = p[1:].copy(), m[1:].copy(), v[1:].copy()
    O.adamw_update(pp, g[1:] * s, mm, vv, 1e-3, 0.9, 0.95, 1e-8, 0.1, b1t, b2t)
    assert bits_equal(bufs[0].numpy()[1:], pp)
    assert bits_equal(bufs[2].numpy()[1:], mm)
    assert bits_equal(bufs[0].numpy()[:1], p[:1])  # untouched


def test_adamw_float32_golden_from_dtrain(dev, golden):
    D, K = _dev()
    G = golden("dtrain_adamw_float32.npz")
    p = D.from_numpy(G["p0"])
    m = D.zeros(p.shape, np.float32)
    v = D.zeros(p.shape, np.float32)
    for k in range(3):
        b1t, b2t = O.bias_corrections(0.9, 0.95, k + 1)
        K.adamw(p, D.from_numpy(G[f"g{k}"]), m, v, 1e-3, 0.9, 0.95, 1e-8, 0.1, b1t, b2t)
        assert bits_equal(p.numpy(), G[f"p{k + 1}"])
        assert bits_equal(m.numpy(), G[f"m{k + 1}"])
        assert bits_equal(v.numpy(), G[f"v{k + 1}"])


@pytest.mark.parametrize("dt", [np.float64, np.float32])
def test_adamw_multi_matches_per_array_loop(dev, dt):
    D, K = _dev()
    rng = np.random.default_rng(9)
    sizes = [5, 64 * 65, 1, 0, 70_000, 33]
    arrs = [_adam_inputs(rng, n, dt) if n > 7 else tuple(a[:n] for a in _adam_inputs(rng, 8, dt)) for n in sizes]
    dps, dgs, dms, dvs = [], [], [], []
    for i, (p, g, m, v) in enumerate(arrs):
        dps.append(D.from_numpy(p))
        dgs.append(None if i == 2 else D.from_numpy(g))  # a parameter without gradient is skipped
        dms.append(D.from_numpy(m))
        dvs.append(D.from_numpy(v))
    b1t, b2t = O.bias_corrections(0.9, 0.95, 7)
    K.adamw_multi(dps, dgs, dms, dvs, 2e-4, 0.9, 0.95, 1e-8, 0.1, b1t, b2t, gscale=0.5)
    for i, (p, g, m, v) in enumerate(arrs):
        p0 = p.copy()
        if i != 2:
            O.adamw_update(p, g * 0.5, m, v, 2e-4, 0.9, 0.95, 1e-8, 0.1, b1t, b2t)
        assert bits_equal(dps[i].numpy(), p), i
        assert bits_equal(dms[i].numpy(), m), i
        if i == 2:
            assert bits_equal(p, p0)


@pytest.mark.parametrize("dt", [np.float64, np.float32])
@pytest.mark.parametrize("world", [1, 2, 3, 4, 5, 8])
@pytest.mark.parametrize("n", [1, 262_144, 1_000_001])
def test_bucket_average_fixed_order_bit_exact(dev, dt, world, n):
    D, K = _dev()
    rng = np.random.default_rng(world * 7 + n)
    reps = (rng.standard_normal((world, n)) * 1e-3).astype(dt)
    out = D.empty((n,), dt)
    nb = K.average_blocks(n, dt)
    parts = D.empty((nb,), np.float64)
    K.bucket_average(out, D.from_numpy(reps), world, 1.0 / world, partials=parts)
    ref = fixed_order_sum(list(reps))
    ref *= 1.0 / world  # dtrain/ddp.py:104-106
    got = out.numpy()
    assert bits_equal(got, ref)
    sq = D.empty((1,), np.float64)
    K.sumsq_finish(parts, nb, sq)
    ref_sq = float(np.dot(ref.astype(np.float64), ref.astype(np.float64)))
    assert abs(float(sq.numpy()[0]) - ref_sq) <= 1e-14 * ref_sq


def test_flatten_aligned_sources_bit_exact(dev):
    """16-byte aligned sources and slots take the vector copy (four vectors in
    flight per thread, then a one-vector loop, then a scalar tail): sizes that
    fill whole chunks, end mid-chunk and end off a multiple of four."""
    D, K = _dev()
    rng = np.random.default_rng(11)
    counts = [40000, 262144, 12, 70004, 5, 4]
    host = [rng.standard_normal(n).astype(np.float32) for n in counts]
    srcs = [D.from_numpy(h) for h in host]
    srcs[3] = None
    dst = D.full((sum(counts),), 9.0, np.float32)
    K.bucket_flatten(dst, srcs, counts)
    ref = np.concatenate([h if i != 3 else np.zeros(counts[3], np.float32) for i, h in enumerate(host)])
    assert bits_equal(dst.numpy(), ref)


def test_flatten_with_missing_grads(dev):
    D, K = _dev()
    rng = np.random.default_rng(3)
    shapes = [(3, 5), (7,), (64, 64), (1,), (1000, 3)]
    host = [rng.standard_normal(s).astype(np.float32) for s in shapes]
    srcs = [D.from_numpy(h) for h in host]
    srcs[1] = None
    counts = [int(np.prod(s)) for s in shapes]
    dst = D.full((sum(counts) + 3,), 9.0, np.float32)
    K.bucket_flatten(dst, [s if s is None else s.reshape(-1) for s in srcs], counts)
    ref = np.concatenate([h.reshape(-1) if i != 1 else np.zeros(counts[1], np.float32) for i, h in enumerate(host)])
    got = dst.numpy()
    assert bits_equal(got[:ref.size], ref)
    assert np.all(got[ref.size:] == 9.0)


@pytest.mark.parametrize("dt", [np.float64, np.float32])
def test_sumsq_deterministic_and_close_to_dtrain(dev, dt):
    D, K = _dev()
    rng = np.random.default_rng(1)
    grads = [(rng.standard_normal(n) * 10.0 ** rng.uniform(-3, 1)).astype(dt) for n in (17, 100_000, 3, 2_000_000)]
    out1, out2 = D.empty((1,), np.float64), D.empty((1,), np.float64)
    dg = [D.from_numpy(g) for g in grads]
    K.sumsq(dg, out1)
    K.sumsq(dg, out2)
    a, b = out1.numpy()[0], out2.numpy()[0]
    assert bits_equal(np.float64(a), np.float64(b))
    ref = O.global_sq_norm(grads)
    assert abs(a - ref) <= 1e-14 * ref


def test_clip_scale_bit_exact_with_dtrain(dev):
    D, K = _dev()
    for sq in (0.0, 0.25, 1.0, 1.0000000001, 4.0, 1234.5678, 1e-300, 7.0e30):
        s_dev, n_dev = D.empty((1,), np.float64), D.empty((1,), np.float64)
        K.clip_scale(D.from_numpy(np.array([sq])), 1.0, s_dev, n_dev)
        assert s_dev.numpy()[0] == O.clip_scale(sq, 1.0), sq
        assert n_dev.numpy()[0] == float(np.sqrt(sq))


@pytest.mark.parametrize("dt", [np.float32, np.float64])
def test_bucket_average_and_adamw_at_124m_params(dev, dt):
    """The gradient-bucket + optimizer workload at full size (124,439,808
    elements, 4 replicas, step 101) in float32 and float64: the fixed-order
    average, the clip factor and AdamW over the full buffer bit-exact against
    the oracle, then AdamW on the 1/4 ZeRO shard [0, 31,109,952) (a view at
    the buffer's start, as rank 0 of dtrain/zero.py:37-39 holds it) from the
    same starting state, bit-exact as well."""
    D, K = _dev()
    n, W = 124_439_808, 4
    rng = np.random.default_rng(4)
    p = (rng.standard_normal(n, dtype=dt) * dt(0.02))
    reps = rng.standard_normal((W, n), dtype=dt) * dt(1e-3)
    m = np.abs(rng.standard_normal(n, dtype=dt) * dt(1e-4))
    v = np.abs(rng.standard_normal(n, dtype=dt) * dt(1e-4))
    sh = n // W
    p_sh, m_sh, v_sh = p[:sh].copy(), m[:sh].copy(), v[:sh].copy()
    dp, dm, dv = D.from_numpy(p), D.from_numpy(m), D.from_numpy(v)
    dg = D.empty((n,), dt)
    nb = K.average_blocks(n, dt)
    parts = D.empty((nb,), np.float64)
    drep = D.from_numpy(reps)
    K.bucket_average(dg, drep, W, 0.25, partials=parts)
    del drep
    sq = D.empty((1,), np.float64)
    K.sumsq_finish(parts, nb, sq)
    s_dev = D.empty((1,), np.float64)
    K.clip_scale(sq, 1.0, s_dev)
    b1t, b2t = O.bias_corrections(0.9, 0.95, 101)
    K.adamw(dp, dg, dm, dv, 3e-4, 0.9, 0.95, 1e-8, 0.1, b1t, b2t, gscale_dev=s_dev)
    # the shard leg: rank 0's slice of a second copy of the starting state
    sp, sm, sv = D.empty((n,), dt), D.empty((n,), dt), D.empty((n,), dt)
    for dst, src in ((sp, p_sh), (sm, m_sh), (sv, v_sh)):
        K.copy_into(dst[:sh], D.from_numpy(src))
    K.adamw(sp[:sh], dg[:sh], sm[:sh], sv[:sh], 3e-4, 0.9, 0.95, 1e-8, 0.1, b1t, b2t, gscale_dev=s_dev)
    g = fixed_order_sum(list(reps))
    del reps
    g *= dt(0.25)
    assert bits_equal(dg.numpy(), g)
    # dtrain's BLAS ddot over 124M terms carries ~1e-13 relative error of its
    # own; judge both against an extended-precision sum of the exact squares.
    g64 = g.astype(np.float64)
    exact = float(np.sum(np.square(g64).astype(np.longdouble)))
    ref_sq = float(np.dot(g64, g64))
    del g64
    got_sq = float(sq.numpy()[0])
    assert abs(got_sq - exact) <= 1e-14 * exact
    assert abs(got_sq - ref_sq) <= 1e-12 * ref_sq
    s = float(s_dev.numpy()[0])
    assert s == O.clip_scale(got_sq, 1.0)
    assert abs(s - O.clip_scale(ref_sq, 1.0)) <= 1e-12
    gs = g * s  # dtrain/train.py:159: the Python float is rounded to the array dtype
    O.adamw_update(p, gs, m, v, 3e-4, 0.9, 0.95, 1e-8, 0.1, b1t, b2t)
    assert bits_equal(dp.numpy(), p)
    assert bits_equal(dm.numpy(), m)
    assert bits_equal(dv.numpy(), v)
    O.adamw_update(p_sh, gs[:sh], m_sh, v_sh, 3e-4, 0.9, 0.95, 1e-8, 0.1, b1t, b2t)
    assert bits_equal(sp.numpy()[:sh], p_sh)
    assert bits_equal(sm.numpy()[:sh], m_sh)
    assert bits_equal(sv.numpy()[:sh], v_sh)
    assert bits_equal(p_sh, p[:sh])


@pytest.mark.parametrize("dt,algo", [(np.float32, "direct"), (np.float64, "direct"), (np.float32, "ring")])
def test_bucket_average_at_124m_params_through_ddp_buckets(dev, dt, algo):
    """The 124,439,808-element, 4-replica average through DDP's 1 MiB bucket
    layout (dtrain/ddp.py:46-56: 474 full buckets and a remainder in float32,
    949 and a remainder in float64) and the merged launches DDP.finish issues
    (ddp.py:84-110): bit-exact to dtrain's bucketed all-reduce in rank order
    ("direct", the workload's fixed order 0..3) or in its ring order, times
    1/4; the norm it leaves within 1e-14 of an extended-precision sum."""
    from dtmi import ddp as P, device as D, replicas as R
    from dtmi.workload import N_BUCKET_WORKLOAD, BucketParams
    from oracle.ddp import ddp_average
    n, W = N_BUCKET_WORKLOAD, 4
    rng = np.random.default_rng(4)
    reps = rng.standard_normal((W, n), dtype=dt) * dt(1e-3)
    model = BucketParams(D.zeros((n,), dt))
    per = (1 << 20) // np.dtype(dt).itemsize
    assert model.sizes[1:] == [per] * (n // per) and model.sizes[0] == n % per
    pg = R.SimGroup(W)
    ddp = P.DDP(model, pg, bucket_mb=1.0, algo=algo)
    assert len(ddp.buckets) == n // per + 1
    ddp.grads.rows.assign(reps)
    launches = []
    average = pg.average
    pg.average = lambda out, rows, **kw: (launches.append(rows.shape[1]), average(out, rows, **kw))
    model.hand_over(ddp)
    assert sum(launches) == n and len(launches) < len(ddp.buckets) // 3
    got = ddp.avg.numpy()[:n]
    if algo == "direct":
        ref = fixed_order_sum(list(reps))
        ref *= dt(0.25)
    else:
        sizes = model.sizes
        offs = np.cumsum([0] + sizes)
        ref = np.concatenate(ddp_average([[reps[r, offs[i]:offs[i + 1]] for i in range(len(sizes))]
                                          for r in range(W)], np.dtype(dt).itemsize, 1.0, algo="ring"))
    assert bits_equal(got, ref)
    for i in (0, len(model.ps) // 2, len(model.ps) - 1):  # the grads are the averaged buffer's slices
        off = sum(model.sizes[:i])
        assert bits_equal(model.ps[i].grad.numpy(), ref[off:off + model.sizes[i]])
    del reps
    r64 = ref.astype(np.float64)
    exact = float(np.sum(np.square(r64).astype(np.longdouble)))
    assert abs(float(ddp.grad_sq.numpy()[0]) - exact) <= 1e-14 * exact


def _ring_ref(reps, segs, dt):
    W, n = reps.shape
    starts = [s for s, _ in segs] + [n]
    out = np.empty(n, dt)
    for j, (s, f) in enumerate(segs):
        acc = reps[f, s:starts[j + 1]].copy()
        for r in range(1, W):
            acc += reps[(f + r) % W, s:starts[j + 1]]
        out[s:starts[j + 1]] = acc
    out *= dt(1.0 / W)  # dtrain/ddp.py:104-106 (weak Python float)
    return out


@pytest.mark.parametrize("dt", [np.float64, np.float32])
@pytest.mark.parametrize("world", [3, 4, 5])
@pytest.mark.parametrize("case", ["one_rotated", "block_edges", "inside_blocks", "many", "large"])
def test_bucket_average_ring_order_bit_exact(dev, dt, world, case):
    """Segments with their own starting rank (dtrain's ring order): whole
    buffer rotated, edges on and inside blocks, more than 16 segments
    (several launches), a 5M-element buffer (blocks of four vectors per
    thread), against a NumPy rank-order sum per segment; gradients over 16
    decades so that any other order changes bits."""
    D, K = _dev()
    rng = np.random.default_rng(world + len(case))
    n = 5_000_003 if case == "large" else 70_001
    reps = (rng.standard_normal((world, n)) * 10.0 ** rng.uniform(-8, 8, (world, n))).astype(dt)
    if case == "one_rotated":
        segs = [(0, world - 1)]
    elif case == "block_edges":
        segs = [(0, 1), (1024, 2), (4096, 0), (40960, world - 1)]
    elif case == "inside_blocks":
        segs = [(0, 2), (5, 1), (1030, 0), (1031, world - 1), (33333, 1), (70_000, 2)]
    elif case == "large":
        segs = [(0, 1), (2048, 0), (4100, 2), (1_666_667, world - 1), (3_333_334, 1), (4_999_999, 0)]
    else:
        cuts = np.sort(rng.choice(np.arange(1, n), 70, replace=False))
        segs = [(0, 1)] + [(int(c), int(rng.integers(0, world))) for c in cuts]
    out = D.full((n,), 7.0, dt)
    K.bucket_average(out, D.from_numpy(reps), world, 1.0 / world, segments=segs)
    ref = _ring_ref(reps, segs, dt)
    assert bits_equal(out.numpy(), ref)
    assert not bits_equal(ref, fixed_order_sum(list(reps)) * dt(1.0 / world))
    if len(segs) <= 16:  # with sum-of-squares partials (one launch)
        nb = K.average_blocks(n, dt)
        parts = D.empty((nb,), np.float64)
        out2 = D.empty((n,), dt)
        K.bucket_average(out2, D.from_numpy(reps), world, 1.0 / world, partials=parts, segments=segs)
        assert bits_equal(out2.numpy(), ref)
        sq = D.empty((1,), np.float64)
        K.sumsq_finish(parts, nb, sq)
        r64 = ref.astype(np.float64)
        ex = float(np.sum(np.square(r64).astype(np.longdouble)))
        assert abs(float(sq.numpy()[0]) - ex) <= 1e-14 * ex


def test_bucket_average_ring_rejects_bad_segments(dev):
    D, K = _dev()
    reps = D.zeros((3, 100), np.float32)
    out = D.empty((100,), np.float32)
    from dtmi._lib import DtmiError
    for segs in ([(1, 0)], [(0, 3)], [(0, 1), (0, 2)], [(0, 1), (100, 2)]):
        with pytest.raises(DtmiError):
            K.bucket_average(out, reps, 3, 1.0 / 3, segments=segs)
