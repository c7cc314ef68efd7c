"""W simulated data-parallel ranks on one GPU.

dtrain runs one process per rank and sums gradients over TCP
(dtrain/comm.py). Here the W ranks are replicas held in one process: each
replica runs its forward/backward in turn on the shared parameters (identical
on every rank, which is what dtrain's broadcast from rank 0 establishes) and
leaves its gradient buckets in its own rows of HBM; the all-reduce becomes one
on-device reduction over the rows in the rank order dtrain's collective would
use: its direct algorithm sums rank 0 first, then 1, 2, ...
(dtrain/comm.py:374-391); its ring (comm.py:292-303, 342-372, the default)
cuts a buffer into partition(n, W) chunks and sums chunk c starting at rank
c, (x_c + x_{c+1}) + ... + x_{c-1}. `ring_segments` maps those chunks onto
this build's layout, so either order gives dtrain's bits.

`SimGroup` stands where dtrain's ProcessGroup stands for DDP and ZeroAdamW:
`.rank` (the replica currently running), `.world`, `broadcast`, `barrier`,
plus the fixed-order reduction itself. Its collectives (`allreduce`,
`allreduce_async`, `reduce_scatter`, `all_gather`) take every rank's buffer
at once -- one process holds them all -- and give each rank the bits dtrain's
collective would leave in that rank's buffer.
"""
from __future__ import annotations

import contextlib

from . import _lib
from . import device as dev
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
        self._after = []

    def set_rank(self, r: int):
        if not 0 <= r < self.world:
            raise ValueError(f"rank {r} out of range for world {self.world}")
        if r != self.rank:
            for fn in self._listeners:
                fn(self.rank)
            self.rank = r
            for fn in self._after:
                fn(r)

    @contextlib.contextmanager
    def replica(self, r: int):
        """Run the enclosed forward/backward as rank r."""
        self.set_rank(r)
        yield self

    def on_rank_change(self, fn):
        """fn(previous_rank) is called before the running replica changes."""
        self._listeners.append(fn)

    def on_rank_set(self, fn):
        """fn(new_rank) is called after the running replica has changed."""
        self._after.append(fn)

    def broadcast(self, arr, root=0):
        """Replicas share one copy of the parameters: identical by construction."""
        return arr

    def barrier(self):
        _lib.sync()

    # ------------------------------------------------ dtrain's collectives
    def _ranks(self, arrays, name):
        arrays = list(arrays)
        if len(arrays) != self.world:
            raise ValueError(f"{name}: need one array per rank ({self.world}), got {len(arrays)}")
        a0 = arrays[0]
        for a in arrays:
            if a.shape != a0.shape or a.dtype != a0.dtype:
                raise ValueError(f"{name}: every rank's array must have the same shape and dtype")
            if not a.is_contiguous:
                raise ValueError(f"{name} needs contiguous arrays")
        return arrays

    def _ordered_sum(self, arrays, firsts):
        """[n] sum over the ranks' arrays, element i summed starting at rank
        firsts(i) (see ring_segments); returns the sum as a new array."""
        n = arrays[0].size
        rows = dev.empty((self.world, max(n, 1)), arrays[0].dtype)
        for r, a in enumerate(arrays):
            if n:
                K.copy_into(rows[r][:n], a.reshape(-1))
        out = dev.empty((n,), arrays[0].dtype)
        if n:
            K.bucket_average(out, rows, self.world, 1.0, segments=firsts)
        return out

    def allreduce(self, arrays, algo: str = "ring"):
        """dtrain/comm.py:292-307, ProcessGroup.allreduce, for all W ranks at
        once: `arrays[r]` is rank r's contiguous array; afterwards every one
        holds the sum over ranks in `algo`'s order -- ring: chunk c of
        partition(n, W) summed starting at rank c, (x_c + x_{c+1}) + ... +
        x_{c-1} (comm.py:342-372); direct: rank 0 first (comm.py:374-391).
        Returns the list."""
        if algo not in ("ring", "direct"):
            raise ValueError(algo)
        arrays = self._ranks(arrays, "allreduce")
        if self.world == 1:
            return arrays
        n = arrays[0].size
        segs = None
        if algo == "ring":
            b = partition(n, self.world)
            segs = [(b[c], c) for c in range(self.world) if b[c] < b[c + 1]] or [(0, 0)]
        total = self._ordered_sum(arrays, segs)
        for a in arrays:
            if n:
                K.copy_into(a.reshape(-1), total)
        return arrays

    def allreduce_async(self, arrays, algo: str = "ring"):
        """comm.py:397-401: the same as allreduce (ordered on the library
        stream); the returned work's wait() returns once it has been issued."""
        self.allreduce(arrays, algo)
        return _Done()

    def reduce_scatter(self, flats):
        """comm.py:309-315 for all W ranks: afterwards partition r of flats[r]
        holds the total of that partition, summed starting at rank r (the
        ring's order with ownership rotated); returns the W partition views.
        The other partitions keep their values (dtrain leaves partial sums
        there, which nothing reads)."""
        flats = self._ranks(flats, "reduce_scatter")
        n = flats[0].size
        b = partition(n, self.world)
        views = [flats[r].reshape(-1)[b[r]:b[r + 1]] for r in range(self.world)]
        if self.world == 1:
            return views
        segs = [(b[c], c) for c in range(self.world) if b[c] < b[c + 1]] or [(0, 0)]
        total = self._ordered_sum(flats, segs)
        for r in range(self.world):
            if b[r] < b[r + 1]:
                K.copy_into(views[r], total[b[r]:b[r + 1]])
        return views

    def all_gather(self, flats):
        """comm.py:317-321 for all W ranks: partition r of flats[r] is copied
        into every rank's flat. Returns the list."""
        flats = self._ranks(flats, "all_gather")
        b = partition(flats[0].size, self.world)
        for r in range(self.world):
            if b[r] == b[r + 1]:
                continue
            src = flats[r].reshape(-1)[b[r]:b[r + 1]]
            for q in range(self.world):
                if q != r:
                    K.copy_into(flats[q].reshape(-1)[b[r]:b[r + 1]], src)
        return flats

    def average(self, out: DeviceArray, rows: DeviceArray, partials: DeviceArray | None = None, segments=None):
        """out = (((rows[0] + rows[1]) + ...) + rows[W-1]) * (1.0 / W), or in
        the rank orders of `segments` ((start, first_rank) pairs, see
        ring_segments)."""
        K.bucket_average(out, rows, self.world, 1.0 / self.world, partials=partials, segments=segments)


class _Done:
    """dtrain's Work (comm.py:229-238) for a collective already issued."""

    def wait(self):
        return None


def ring_segments(sizes, world: int):
    """Where dtrain's ring chunks fall in this build's bucket layout.

    dtrain concatenates a bucket's parameters in REVERSE definition order
    (dtrain/ddp.py:27-37, 46-56) and its ring all-reduce sums chunk c of
    partition(n, W) of that buffer starting at rank c (comm.py:342-372). Here
    the same parameters sit in forward order. `sizes` are the bucket's
    parameter sizes in forward order; returns (start, first_rank) pairs in
    ascending start over the forward-order buffer (consecutive pieces with the
    same first rank merged): element i is summed starting at the first_rank
    of the last pair whose start <= i."""
    n = sum(sizes)
    bounds = partition(n, world)
    # offset of each parameter in dtrain's (reversed) buffer
    dofs, off = [0] * len(sizes), 0
    for i in reversed(range(len(sizes))):
        dofs[i] = off
        off += sizes[i]
    segs = []
    o = 0
    for i, k in enumerate(sizes):
        a, b = dofs[i], dofs[i] + k
        for c in range(world):
            lo, hi = max(a, bounds[c]), min(b, bounds[c + 1])
            if lo < hi and (not segs or segs[-1][1] != c):
                segs.append((o + lo - a, c))
        o += k
    return segs or [(0, 0)]


class ReplicaGrads:
    """Every replica's gradients in HBM: a [W, n] buffer, one row per replica,
    each row holding all parameters' gradients back to back in forward
    (definition) order.

    The running replica's slot for each parameter is installed as that
    parameter's `grad_dest`, so the backward kernels that produce parameter
    gradients (Linear dW/db, LayerNorm dgamma/dbeta, the embedding table)
    write them straight into the row: the copy dtrain makes to fill its
    buckets (ddp.py:73-81, zero.py:46-53) is needed only for a gradient that
    did not land in its slot (`place`). Slots of parameters that received no
    gradient are zero-filled (`zero`).
    """

    def __init__(self, params, pg: "SimGroup", dtype):
        self.params = list(params)
        self.pg = pg
        self.offsets = []
        off = 0
        for p in self.params:
            self.offsets.append(off)
            off += p.data.size
        self.n = off
        self.rows = dev.empty((pg.world, max(off, 1)), dtype)
        self.index = {id(p): i for i, p in enumerate(self.params)}
        self._dest = [[self.rows[r][o:o + p.data.size].reshape(p.data.shape)
                       for p, o in zip(self.params, self.offsets)] for r in range(pg.world)]
        self.attach(pg.rank)
        pg.on_rank_set(self.attach)

    def attach(self, r: int):
        for p, d in zip(self.params, self._dest[r]):
            p.grad_dest = d

    def slot(self, r: int, i: int) -> DeviceArray:
        return self._dest[r][i]

    def place(self, r: int, i: int, g: DeviceArray):
        """Make replica r's slot i hold g (a copy unless g already is the slot)."""
        d = self._dest[r][i]
        if g.ptr != d.ptr:
            K.copy_into(d, g)

    def zero(self, r: int, i: int):
        self._dest[r][i].zero_()

    def columns(self, lo: int, hi: int) -> DeviceArray:
        """The [W, hi - lo] view of columns lo..hi of every replica's row."""
        isz = self.rows.itemsize
        return DeviceArray(self.rows.block, (self.pg.world, hi - lo), self.rows.dtype, self.rows.offset + lo * isz,
                           (self.rows.strides[0], 1))
