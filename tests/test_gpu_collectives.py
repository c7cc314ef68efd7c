"""SimGroup's collectives, dtrain's ProcessGroup API (dtrain/comm.py:292-321,
397-401) over the W simulated ranks' buffers at once, against the oracle's
rank orders (pinned by dtrain's own DDP and ZeroAdamW fixtures): bit-exact,
with values over 16 decades so that any other summation order changes bits.
The cases follow dtrain's tests/test_comm.py (all-reduce against a sum for
both algorithms, reduce-scatter then all-gather over ragged partitions)."""
import numpy as np
import pytest

from helpers import bits_equal
from oracle.ddp import allreduce_sum, partition, ring_order_sum

pytestmark = pytest.mark.gpu


def _api():
    from dtmi import device as D, replicas as R
    return D, R


def _parts(world, n, dt, seed):
    rng = np.random.default_rng(seed)
    return [(rng.standard_normal(n) * 10.0 ** rng.uniform(-8, 8, n)).astype(dt) for _ in range(world)]


@pytest.mark.parametrize("dt", [np.float64, np.float32])
@pytest.mark.parametrize("algo", ["ring", "direct"])
@pytest.mark.parametrize("world", [1, 2, 3, 4, 5])
@pytest.mark.parametrize("n", [1, 3, 1000, 70_001])
def test_allreduce_matches_dtrains_order(dev, dt, algo, world, n):
    D, R = _api()
    parts = _parts(world, n, dt, world * 7 + n)
    pg = R.SimGroup(world)
    bufs = [D.from_numpy(p) for p in parts]
    pg.allreduce(bufs, algo)
    ref = allreduce_sum(parts, algo)
    for b in bufs:
        assert bits_equal(b.numpy(), ref)
    if world >= 3 and n >= 1000:
        other = allreduce_sum(parts, "direct" if algo == "ring" else "ring")
        assert not bits_equal(ref, other)  # the two orders are told apart


def test_allreduce_async_and_multidimensional(dev):
    D, R = _api()
    parts = _parts(4, 6 * 50, np.float32, 3)
    pg = R.SimGroup(4)
    bufs = [D.from_numpy(p.reshape(6, 50)) for p in parts]
    w = pg.allreduce_async(bufs)
    assert w.wait() is None
    ref = ring_order_sum(parts).reshape(6, 50)
    for b in bufs:
        assert bits_equal(b.numpy(), ref)


@pytest.mark.parametrize("dt", [np.float64, np.float32])
@pytest.mark.parametrize("world", [1, 2, 3, 4])
@pytest.mark.parametrize("n", [2, 10, 1001])
def test_reduce_scatter_then_all_gather(dev, dt, world, n):
    """Partition r of rank r's buffer holds the total of partition r (summed
    starting at rank r); after the all-gather every rank holds every total."""
    D, R = _api()
    parts = _parts(world, n, dt, n + world)
    pg = R.SimGroup(world)
    flats = [D.from_numpy(p) for p in parts]
    views = pg.reduce_scatter(flats)
    total = ring_order_sum(parts) if world > 1 else parts[0]
    b = partition(n, world)
    for r in range(world):
        assert bits_equal(views[r].numpy(), total[b[r]:b[r + 1]])
    pg.all_gather(flats)
    for f in flats:
        assert bits_equal(f.numpy(), total)


def test_collectives_reject_bad_arguments(dev):
    D, R = _api()
    pg = R.SimGroup(3)
    a = [D.zeros((4,), np.float32) for _ in range(2)]
    with pytest.raises(ValueError):
        pg.allreduce(a)  # one array per rank
    with pytest.raises(ValueError):
        pg.allreduce([D.zeros((4,), np.float32) for _ in range(3)], algo="tree")
    with pytest.raises(ValueError):
        pg.reduce_scatter([D.zeros((4,), np.float32), D.zeros((5,), np.float32), D.zeros((4,), np.float32)])
