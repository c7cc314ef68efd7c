"""Distributed data parallel with gradient buckets over W simulated replicas.

dtrain/ddp.py on one GPU. Same constructor, attributes and step protocol:

* parameters are "broadcast" from rank 0 at construction (replicas share one
  parameter copy, so they are identical by construction);
* parameters are grouped into buckets of about `bucket_mb` MiB in reverse
  definition order, closing a bucket as soon as it reaches the limit
  (ddp.py:46-56);
* a grad-ready hook on every parameter hands its gradient to the bucket; when
  all of a bucket's gradients of the running replica are in, one multi-tensor
  flatten kernel copies them into that replica's row of the bucket (ddp.py:73-81
  copies one parameter at a time); when the last replica's row is complete the
  fixed-order average of the bucket is launched right away (`overlap=True`) or
  at `finish()` (`overlap=False`);
* `no_sync()` skips all of this for gradient-accumulation micro-steps;
* `finish()` zero-fills missing gradients (ddp.py:88-94), reduces what is left,
  and points every `param.grad` at its slice of the averaged bucket
  (ddp.py:104-110). The average is
  (((g_0 + g_1) + g_2) + ... + g_{W-1}) * (1.0 / W), dtrain's `--algo direct`
  order (comm.py:374-391), bit-exact to NumPy. The same kernel accumulates
  the squares of the averaged gradients per block; `grad_sq` (a 1-element
  float64 device array) is their deterministic sum after `finish()`, the
  global-norm input of dtrain/train.py:155-156 without another pass.

The ring order of dtrain's default `--algo ring` (each chunk starts at a
different rank, comm.py:342-372) is not reproduced; see the module docstring
of dtmi.replicas.
"""
from __future__ import annotations

import contextlib
import time

import numpy as np

from . import device as dev
from . import kernels as K
from .device import DeviceArray


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
    def __init__(self, params, dtype, world):
        self.params = params
        self.offsets = []
        off = 0
        for p in params:
            self.offsets.append(off)
            off += p.data.size
        self.n = off
        self.rows = dev.empty((world, off), dtype)  # one row per replica (dtrain's b.buf, per rank)
        self.ready = [dict() for _ in range(world)]
        self.pending = [len(params)] * world
        self.flushed = [False] * world
        self.out = None  # averaged gradients of the last reduction
        self.reduced = False
        self.partial_off = 0
        self.nblocks = K.average_blocks(off) if off else 0

    @property
    def buf(self) -> DeviceArray:
        """The averaged bucket after finish() (dtrain's b.buf after `*= 1/W`)."""
        return self.out


class DDP:
    def __init__(self, model, pg, bucket_mb: float = 1.0, overlap: bool = True, algo: str = "direct"):
        if algo not in ("direct", "ring"):
            raise ValueError(f"unknown algo {algo!r}")
        self.model, self.pg, self.overlap, self.algo = model, pg, overlap, algo
        self.params = model.parameters()
        for p in self.params:
            pg.broadcast(p.data, root=0)
        dtype = self.params[0].data.dtype
        sizes = [p.data.size for p in self.params]
        self.buckets = [_Bucket([self.params[i] for i in idx], dtype, pg.world)
                        for idx in bucket_layout(sizes, np.dtype(dtype).itemsize, bucket_mb)]
        self._where = {}
        off = 0
        for bi, b in enumerate(self.buckets):
            b.partial_off = off
            off += b.nblocks
            for pi, p in enumerate(b.params):
                self._where[id(p)] = (bi, pi)
                p.register_grad_ready_hook(self._on_grad)
        self._partials = dev.empty((max(off, 1),), np.float64)
        self._nparts = off
        self._sync = True
        self.comm_wait_s = 0.0
        self.grad_sq = None

    @contextlib.contextmanager
    def no_sync(self):
        prev, self._sync = self._sync, False
        try:
            yield
        finally:
            self._sync = prev

    def _flatten(self, b: _Bucket, r: int):
        srcs = []
        for pi, p in enumerate(b.params):
            g = b.ready[r].get(pi)
            if g is not None and not g.is_contiguous:
                g = g.contiguous()
            srcs.append(g.reshape(-1) if g is not None else None)  # missing: zeros (ddp.py:88-94)
        K.bucket_flatten(b.rows[r], srcs, [p.data.size for p in b.params])
        b.ready[r].clear()
        b.flushed[r] = True

    def _reduce(self, b: _Bucket):
        if b.reduced or b.n == 0:
            b.reduced = True
            return
        b.out = dev.empty((b.n,), b.rows.dtype)
        parts = self._partials[b.partial_off:b.partial_off + b.nblocks]
        self.pg.average(b.out, b.rows, partials=parts)
        b.reduced = True

    def _on_grad(self, p):
        if not self._sync:
            return
        r = self.pg.rank
        bi, pi = self._where[id(p)]
        b = self.buckets[bi]
        if pi not in b.ready[r]:
            b.pending[r] -= 1
        b.ready[r][pi] = p.grad
        if b.pending[r] == 0:
            self._flatten(b, r)
            if self.overlap and all(b.flushed):
                self._reduce(b)

    def finish(self):
        """Complete gradient synchronisation; call after the last backward of a step."""
        t0 = time.perf_counter()
        W = self.pg.world
        for b in self.buckets:
            for r in range(W):
                if not b.flushed[r]:
                    self._flatten(b, r)
            self._reduce(b)
        self.grad_sq = dev.empty((1,), np.float64)
        K.sumsq_finish(self._partials, self._nparts, self.grad_sq)
        for b in self.buckets:
            for pi, p in enumerate(b.params):
                off = b.offsets[pi]
                p.grad = b.out[off:off + p.data.size].reshape(p.data.shape)
            b.pending = [len(b.params)] * W
            b.flushed = [False] * W
            b.reduced = False
        self.comm_wait_s += time.perf_counter() - t0
