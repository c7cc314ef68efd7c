"""W simulated data-parallel ranks on one GPU.

dtrain runs one process per rank and sums gradients over TCP
(dtrain/comm.py). Here the W ranks are replicas held in one process: each
replica runs its forward/backward in turn on the shared parameters (identical
on every rank, which is what dtrain's broadcast from rank 0 establishes) and
leaves its gradient buckets in its own rows of HBM; the all-reduce becomes one
fixed-order on-device reduction over the rows, in dtrain's direct-algorithm
order (rank 0 first, then 1, 2, ...; dtrain/comm.py:374-391).

`SimGroup` stands where dtrain's ProcessGroup stands for DDP and ZeroAdamW:
`.rank` (the replica currently running), `.world`, `broadcast`, `barrier`,
plus the fixed-order reduction itself.
"""
from __future__ import annotations

import contextlib

from . import _lib
from . import kernels as K
from .device import DeviceArray


def partition(n: int, world: int):
    """dtrain/comm.py:220-226: rank r owns [b[r], b[r+1]); the first n % W
    ranks get one extra element."""
    base, extra = divmod(n, world)
    b = [0]
    for r in range(world):
        b.append(b[-1] + base + (1 if r < extra else 0))
    return b


class SimGroup:
    def __init__(self, world: int):
        if world < 1:
            raise ValueError("world must be >= 1")
        self.world = world
        self.rank = 0
        self._listeners = []

    def set_rank(self, r: int):
        if not 0 <= r < self.world:
            raise ValueError(f"rank {r} out of range for world {self.world}")
        if r != self.rank:
            for fn in self._listeners:
                fn(self.rank)
        self.rank = r

    @contextlib.contextmanager
    def replica(self, r: int):
        """Run the enclosed forward/backward as rank r."""
        self.set_rank(r)
        yield self

    def on_rank_change(self, fn):
        """fn(previous_rank) is called before the running replica changes."""
        self._listeners.append(fn)

    def broadcast(self, arr, root=0):
        """Replicas share one copy of the parameters: identical by construction."""
        return arr

    def barrier(self):
        _lib.sync()

    def average(self, out: DeviceArray, rows: DeviceArray, partials: DeviceArray | None = None):
        """out = (((rows[0] + rows[1]) + ...) + rows[W-1]) * (1.0 / W)."""
        K.bucket_average(out, rows, self.world, 1.0 / self.world, partials=partials)
