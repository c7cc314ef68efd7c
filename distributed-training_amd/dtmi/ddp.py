"""Distributed data parallel with gradient buckets over W simulated replicas.

dtrain/ddp.py on one GPU. Same constructor, attributes and step protocol:

* parameters are "broadcast" from rank 0 at construction (replicas share one
  parameter copy, so they are identical by construction);
* parameters are grouped into buckets of about `bucket_mb` MiB in reverse
  definition order, closing a bucket as soon as it reaches the limit
  (ddp.py:46-56);
* a grad-ready hook on every parameter hands its gradient to the bucket; when
  all of a bucket's gradients of the last replica are in, the fixed-order
  average of the bucket is launched right away (`overlap=True`; a run of
  adjacent buckets that complete one after another shares one launch, up to
  MERGE_BYTES) or at `finish()` (`overlap=False`);
* `no_sync()` skips all of this for gradient-accumulation micro-steps;
* `finish()` zero-fills missing gradients (ddp.py:88-94), reduces what is left,
  and points every `param.grad` at its slice of the averaged gradients
  (ddp.py:104-110). The average is the rank-order sum times (1.0 / W), in
  the order of dtrain's all-reduce for `algo`: "ring" (its default: chunk c
  of partition(n, W) of a bucket's buffer summed starting at rank c,
  comm.py:292-303, 342-372) or "direct" ((((g_0 + g_1) + g_2) + ...),
  comm.py:374-391), bit-exact to NumPy either way. `grad_sq` (a 1-element
  float64 device array) is the deterministic float64 sum of squares of all
  averaged gradients after `finish()`, the global-norm input of
  dtrain/train.py:155-156. It is one pass over the flat averaged buffer, so
  neither it nor the clip factor depends on the bucket size.

Memory layout. A bucket is a run of consecutive parameters, so in forward
order it is one contiguous range [lo, hi) of the flat parameter numbering.
Every replica's gradients live in one [W, n] buffer (`ReplicaGrads`) in
forward order, and the backward kernels write each parameter's gradient
straight into its slot there (no flatten copy); bucket b's "buffer" of
replica r is row r, columns [lo, hi). The averaged gradients go to one [n]
buffer in the same order, so after `finish()` the `param.grad` views are
back to back and the optimizer runs as one flat launch. Element order inside
a bucket differs from dtrain's concatenation order (reverse definition
order); the reduction is elementwise, and for the ring order each bucket
carries where dtrain's chunks fall in this layout (dtmi.replicas.
ring_segments), so no value changes.
"""
from __future__ import annotations

import contextlib
import time

import numpy as np

from . import device as dev
from . import kernels as K
from .device import DeviceArray
from .replicas import ReplicaGrads, ring_segments


def bucket_layout(sizes, itemsize, bucket_mb=1.0):
    """Greedy buckets over parameters in reverse order (dtrain/ddp.py:46-56).
    Returns a list of buckets, each a list of parameter indices."""
    limit = int(bucket_mb * (1 << 20))
    buckets, cur, size = [], [], 0
    for i in reversed(range(len(sizes))):
        cur.append(i)
        size += sizes[i] * itemsize
        if size >= limit:
            buckets.append(cur)
            cur, size = [], 0
    if cur:
        buckets.append(cur)
    return buckets


class _Bucket:
    def __init__(self, idx, grads: ReplicaGrads, avg: DeviceArray, algo: str):
        self.idx = idx  # parameter indices, reverse definition order (dtrain's bucket order)
        self.params = [grads.params[i] for i in idx]
        self.lo = grads.offsets[min(idx)]
        self.hi = grads.offsets[max(idx)] + grads.params[max(idx)].data.size
        self.n = self.hi - self.lo
        self.rows = grads.columns(self.lo, self.hi)  # [W, n]: every replica's gradients of this bucket
        self.out = avg[self.lo:self.hi]  # averaged gradients of this bucket
        world = grads.pg.world
        # rank orders of the all-reduce over this bucket (None: rank 0 first)
        self.segments = None
        if algo == "ring" and world > 2:
            self.segments = ring_segments([grads.params[i].data.size for i in sorted(idx)], world)
        self.ready = [set() for _ in range(world)]
        self.flushed = [False] * world
        self.reduced = False

    @property
    def buf(self) -> DeviceArray:
        """The averaged bucket after finish() (dtrain's b.buf after `*= 1/W`)."""
        return self.out


class DDP:
    def __init__(self, model, pg, bucket_mb: float = 1.0, overlap: bool = True, algo: str = "ring"):
        if algo not in ("direct", "ring"):
            raise ValueError(f"unknown algo {algo!r}")
        self.model, self.pg, self.overlap, self.algo = model, pg, overlap, algo
        self.params = model.parameters()
        for p in self.params:
            pg.broadcast(p.data, root=0)
        dtype = self.params[0].data.dtype
        sizes = [p.data.size for p in self.params]
        self.grads = ReplicaGrads(self.params, pg, dtype)
        self.avg = dev.empty((max(self.grads.n, 1),), dtype)
        self.buckets = [_Bucket(idx, self.grads, self.avg, algo)
                        for idx in bucket_layout(sizes, np.dtype(dtype).itemsize, bucket_mb)]
        self._where = {}
        for bi, b in enumerate(self.buckets):
            for i in b.idx:
                self._where[id(self.params[i])] = (bi, i)
        for p in self.params:
            p.register_grad_ready_hook(self._on_grad)
        self._sync = True
        self._pend = []
        self.comm_wait_s = 0.0
        self.grad_sq = None

    @contextlib.contextmanager
    def no_sync(self):
        prev, self._sync = self._sync, False
        try:
            yield
        finally:
            self._sync = prev

    def _complete(self, b: _Bucket, r: int):
        """Zero-fill replica r's slots of the bucket that received no gradient."""
        for i in b.idx:
            if i not in b.ready[r]:
                self.grads.zero(r, i)  # missing: zeros (ddp.py:88-94)
        b.ready[r].clear()
        b.flushed[r] = True

    # Buckets that complete one after another are adjacent column ranges
    # (reverse parameter order), so a run of them is averaged by one launch
    # once it holds MERGE_BYTES of gradients, or at finish(): the average is
    # elementwise with each element's own rank order, so the grouping changes
    # no value, and a 1 MiB bucket alone is too short a launch to reach the
    # memory bandwidth. The replicas share one GPU and one stream, so an
    # earlier launch would overlap nothing: runs are as long as the rank-order
    # segments allow. MAX_SEGS: the rank-order segments one launch takes.
    MERGE_BYTES = 256 << 20
    MAX_SEGS = 16

    def _reduce(self, b: _Bucket):
        if b.reduced or b.n == 0:
            b.reduced = True
            return
        p = self._pend
        if p:
            lo, hi = min(x.lo for x in p), max(x.hi for x in p)
            # rank-order segments of the run (rank-0-first buckets carry none)
            nseg = sum(len(x.segments) for x in p + [b] if x.segments)
            if not (b.hi == lo or b.lo == hi) or nseg > self.MAX_SEGS:
                self._flush()
        self._pend.append(b)
        b.reduced = True
        if sum(x.n for x in self._pend) * self.avg.itemsize >= self.MERGE_BYTES:
            self._flush()

    def _flush(self):
        """Average the pending run of adjacent buckets in one launch."""
        p = sorted(self._pend, key=lambda x: x.lo)
        self._pend = []
        if not p:
            return
        lo, hi = p[0].lo, p[-1].hi
        segs = None
        if any(x.segments for x in p):
            segs = []
            for x in p:
                for st, first in x.segments or ((0, 0),):
                    if not segs or segs[-1][1] != first:
                        segs.append((x.lo - lo + st, first))
        self.pg.average(self.avg[lo:hi], self.grads.columns(lo, hi), segments=segs)

    def _on_grad(self, p):
        if not self._sync:
            return
        r = self.pg.rank
        bi, i = self._where[id(p)]
        b = self.buckets[bi]
        self.grads.place(r, i, p.grad)
        b.ready[r].add(i)
        if len(b.ready[r]) == len(b.idx):
            b.ready[r].clear()
            b.flushed[r] = True
            if self.overlap and all(b.flushed):
                self._reduce(b)

    def finish(self):
        """Complete gradient synchronisation; call after the last backward of a step."""
        t0 = time.perf_counter()
        W = self.pg.world
        for b in self.buckets:
            for r in range(W):
                if not b.flushed[r]:
                    self._complete(b, r)
            self._reduce(b)
        self._flush()
        self.grad_sq = dev.empty((1,), np.float64)
        K.sumsq([self.avg[:self.grads.n]], self.grad_sq)
        for p, o in zip(self.params, self.grads.offsets):
            p.grad = self.avg[o:o + p.data.size].reshape(p.data.shape)
        for b in self.buckets:
            b.flushed = [False] * W
            b.reduced = False
        self.comm_wait_s += time.perf_counter() - t0
