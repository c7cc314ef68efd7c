"""ZeRO-1 sharded AdamW over W simulated replicas (dtrain/zero.py on one GPU).

All parameters live in one contiguous device buffer in forward order and each
parameter's `.data` is a view into it (zero.py:29-35); the buffer is
partitioned with dtrain's `partition` and rank r owns flat[b[r]:b[r+1]]
(`.shard`, `.bounds`). Each replica's backward flattens its gradients into its
own row of a [W, n] buffer in forward order: the backward kernels write
each gradient straight into its slot (see dtmi.replicas.ReplicaGrads), where
zero.py:46-53 flattens after backward. `step()` then, for every shard in rank
order: the sum of the replicas' rows times 1/W (the reduce-scatter plus
`g *= 1/W` of zero.py:54-55, in the order of dtrain's ring reduce-scatter,
comm.py:342-363: shard r is summed starting at rank r,
(x_r + x_{r+1}) + ... + x_{r-1}), its float64 sum of squares, summed over
shards in rank order (the all-reduce of zero.py:56-57); the clip factor
(computed on the device); and AdamW on every shard. AdamW is elementwise, so
one launch over the whole buffer with one m/v buffer gives the same bits as W
per-shard optimizers; `.opt` exposes the running rank's shard view of it, and
`state_bytes()` is that rank's 2 * itemsize * shard size, as in dtrain. The
all-gather (zero.py:62) is free: the shards are slices of the one buffer.
"""
from __future__ import annotations

import numpy as np

from . import device as dev
from . import kernels as K
from .device import DeviceArray
from .optim import AdamW, clip_scale_device
from .replicas import ReplicaGrads, partition


class _ShardOpt:
    """The AdamW state of one rank's shard (views into the shared buffers)."""

    def __init__(self, full: AdamW, lo: int, hi: int):
        self._full, self.lo, self.hi = full, lo, hi

    @property
    def t(self):
        return self._full.t

    @property
    def lr(self):
        return self._full.lr

    @lr.setter
    def lr(self, v):
        self._full.lr = v

    @property
    def m(self):
        return [self._full.m[0][self.lo:self.hi]]

    @property
    def v(self):
        return [self._full.v[0][self.lo:self.hi]]

    def state_bytes(self):
        return 2 * (self.hi - self.lo) * np.dtype(self._full.m[0].dtype).itemsize

    def state_dict(self):
        return {"t": self.t, "m": [a.numpy() for a in self.m], "v": [a.numpy() for a in self.v]}

    def load_state_dict(self, s):
        self._full.t = int(s["t"])
        self.m[0].assign(s["m"][0])
        self.v[0].assign(s["v"][0])


class ZeroAdamW:
    def __init__(self, model, pg, max_grad_norm: float | None = None, **adam):
        self.pg = pg
        self.params = model.parameters()
        n = sum(p.data.size for p in self.params)
        dtype = self.params[0].data.dtype
        self.flat = dev.empty((n,), dtype)
        off = 0
        for p in self.params:
            k = p.data.size
            view = self.flat[off:off + k].reshape(p.data.shape)
            K.copy_into(view, p.data)
            p.data = view  # view into the flat buffer
            off += k
        pg.broadcast(self.flat, root=0)
        self.n = n
        self.bounds = partition(n, pg.world)
        self.grads = ReplicaGrads(self.params, pg, dtype)
        self.gflat = self.grads.rows  # [W, n]: each replica's gradients in forward order
        self._full = AdamW([self.flat], **adam)
        self.opts = [_ShardOpt(self._full, self.bounds[r], self.bounds[r + 1]) for r in range(pg.world)]
        self.max_grad_norm = max_grad_norm
        self._norm = None
        self._ready = [set() for _ in range(pg.world)]
        self._index = self.grads.index
        for p in self.params:
            p.register_grad_ready_hook(self._on_grad)
        self._nblocks = [K.average_blocks(self.bounds[r + 1] - self.bounds[r], dtype) for r in range(pg.world)]
        self._partials = dev.empty((max(1, max(self._nblocks)),), np.float64)

    # dtrain attributes
    @property
    def shard(self) -> DeviceArray:
        r = self.pg.rank
        return self.flat[self.bounds[r]:self.bounds[r + 1]]

    @property
    def opt(self):
        return self.opts[self.pg.rank]

    @property
    def last_grad_norm(self) -> float:
        return 0.0 if self._norm is None else float(self._norm.numpy()[0])

    @property
    def last_grad_norm_device(self):
        return self._norm

    def _on_grad(self, p):
        r, i = self.pg.rank, self._index[id(p)]
        self.grads.place(r, i, p.grad)
        self._ready[r].add(i)

    def _complete(self, r):
        for i in range(len(self.params)):
            if i not in self._ready[r]:
                self.grads.zero(r, i)  # zero.py:49-50
        self._ready[r].clear()

    def step(self):
        W = self.pg.world
        for r in range(W):
            self._complete(r)
        g = dev.empty((self.n,), self.flat.dtype)
        sq = dev.empty((1,), np.float64)
        isz = np.dtype(self.flat.dtype).itemsize
        for r in range(W):  # reduce-scatter + 1/W, shard sum of squares, all-reduce: rank order
            lo, hi = self.bounds[r], self.bounds[r + 1]
            if hi > lo:
                rows = DeviceArray(self.gflat.block, (W, hi - lo), self.gflat.dtype, self.gflat.offset + lo * isz,
                                   (self.n, 1))
                parts = self._partials[:self._nblocks[r]]
                K.bucket_average(g[lo:hi], rows, W, 1.0 / W, partials=parts, segments=[(0, r)])
                K.sumsq_finish(parts, self._nblocks[r], sq, accumulate=r > 0)
            elif r == 0:
                sq.zero_()
        scale, norm = clip_scale_device(sq, self.max_grad_norm if self.max_grad_norm else float("inf"))
        self._norm = norm
        self._full.step([g], grad_scale=scale if self.max_grad_norm else 1.0)

    def state_bytes(self):
        return self.opt.state_bytes()

    def state_dict(self):
        return self.opt.state_dict()

    def load_state_dict(self, s):
        self.opt.load_state_dict(s)
