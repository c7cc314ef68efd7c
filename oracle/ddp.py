"""DDP bucket layout, flatten and fixed-order average; ZeRO partition and step;
restated from dtrain/ddp.py, dtrain/zero.py and dtrain/comm.py for W simulated
ranks held in one process. Both of dtrain's all-reduce orders are restated:
"direct" (rank 0 first) and "ring" (chunk c of a buffer summed starting at
rank c). Test infrastructure only."""
from __future__ import annotations

import numpy as np

from .optim import AdamW, clip_scale


def partition(n: int, world: int):
    """dtrain/comm.py:220-226: rank r owns [b[r], b[r+1]); the first n % W ranks
    get one extra element."""
    base, extra = divmod(n, world)
    b = [0]
    for r in range(world):
        b.append(b[-1] + base + (1 if r < extra else 0))
    return b


def bucket_layout(sizes, itemsize, bucket_mb=1.0):
    """dtrain/ddp.py:46-56: walk parameters in REVERSE order, close a bucket as
    soon as its byte size reaches int(bucket_mb * 2**20). Returns a list of
    buckets, each a list of (param_index, offset_in_bucket, size)."""
    limit = int(bucket_mb * (1 << 20))
    buckets, cur, nbytes = [], [], 0
    for i in reversed(range(len(sizes))):
        cur.append(i)
        nbytes += sizes[i] * itemsize
        if nbytes >= limit:
            buckets.append(cur)
            cur, nbytes = [], 0
    if cur:
        buckets.append(cur)
    out = []
    for b in buckets:
        off, entries = 0, []
        for i in b:
            entries.append((i, off, sizes[i]))
            off += sizes[i]
        out.append(entries)
    return out


def fixed_order_sum(parts):
    """dtrain/comm.py:388-391 (_direct_allreduce): out = parts[0].copy();
    out += parts[1]; ... in rank order."""
    out = parts[0].copy()
    for p in parts[1:]:
        out += p
    return out


def ring_order_sum(parts):
    """dtrain/comm.py:292-303 with 342-372 (ring all-reduce, reduce-scatter
    without the ownership rotation, then all-gather): the buffer is cut into
    partition(n, W) chunks; chunk c travels the ring from rank c, and each hop
    adds the receiving rank's own chunk to what arrived (`flat[ri] += recv`,
    commutative), so chunk c is ((x_c + x_{c+1}) + ...) + x_{c-1}."""
    W = len(parts)
    out = parts[0].copy()
    b = partition(out.size, W)
    for c in range(W):
        lo, hi = b[c], b[c + 1]
        acc = parts[c][lo:hi].copy()
        for j in range(1, W):
            acc += parts[(c + j) % W][lo:hi]
        out[lo:hi] = acc
    return out


def allreduce_sum(parts, algo):
    """ProcessGroup.allreduce (dtrain/comm.py:292-308) for W ranks' buffers."""
    if len(parts) == 1:
        return parts[0].copy()
    if algo == "ring":
        return ring_order_sum(parts)
    if algo == "direct":
        return fixed_order_sum(parts)
    raise ValueError(algo)


def ddp_average(replica_grads, itemsize, bucket_mb=1.0, algo="direct"):
    """DDP.finish (dtrain/ddp.py:84-110) for W replicas' gradient lists: flatten
    each replica into its buckets (hook copy, ddp.py:73-81; missing grads
    contribute zeros, ddp.py:88-94), all-reduce each bucket with `algo`
    ("direct": rank order; "ring": dtrain's default, chunk c of the bucket
    starting at rank c), multiply by 1.0/W, slice back. Returns the averaged
    grads."""
    W = len(replica_grads)
    first = replica_grads[0]
    sizes = [g.size for g in first]
    dtype = first[0].dtype
    layout = bucket_layout(sizes, itemsize, bucket_mb)
    out = [None] * len(sizes)
    inv = 1.0 / W
    for entries in layout:
        n = sum(s for _, _, s in entries)
        bufs = []
        for r in range(W):
            buf = np.zeros(n, dtype)
            for i, off, s in entries:
                g = replica_grads[r][i]
                if g is not None:
                    buf[off:off + s] = g.reshape(-1)
            bufs.append(buf)
        red = allreduce_sum(bufs, algo)
        red *= inv
        for i, off, s in entries:
            out[i] = red[off:off + s].reshape(first[i].shape).copy()
    return out


class ZeroAdamW:
    """dtrain/zero.py:23-62 for W simulated ranks: one flat parameter buffer in
    forward order, shard r = flat[b[r]:b[r+1]], one AdamW per shard. `step`
    takes every replica's flat gradient; the reduce-scatter is dtrain's ring
    (comm.py:310-316, 342-363: after the ownership rotation rank r holds chunk
    r, which the ring summed starting at rank r), then *= 1/W, float64 sum of
    squares per shard summed in rank order (the sq all-reduce: a 1-element
    ring all-reduce is chunk 0, rank order), clip, AdamW."""

    def __init__(self, params, world, max_grad_norm=None, **adam):
        self.world = world
        n = sum(p.size for p in params)
        self.flat = np.concatenate([p.reshape(-1) for p in params]).astype(params[0].dtype)
        self.bounds = partition(n, world)
        self.opts = [AdamW([self.flat[self.bounds[r]:self.bounds[r + 1]]], **adam) for r in range(world)]
        self.max_grad_norm = max_grad_norm
        self.last_grad_norm = 0.0

    def step(self, replica_flat_grads):
        W = self.world
        shards = []
        for r in range(W):
            lo, hi = self.bounds[r], self.bounds[r + 1]
            g = replica_flat_grads[r][lo:hi].copy()
            for j in range(1, W):
                g += replica_flat_grads[(r + j) % W][lo:hi]
            g *= 1.0 / W
            shards.append(g)
        sqs = [float(np.dot(g.astype(np.float64), g.astype(np.float64))) for g in shards]
        sq = np.zeros(1)
        for s in sqs:  # all-reduce of the per-rank sums, rank order
            sq[0] += s
        self.last_grad_norm = float(np.sqrt(sq[0]))
        if self.max_grad_norm:
            s = clip_scale(sq[0], self.max_grad_norm)
            for g in shards:
                g *= s
        for r in range(W):
            self.opts[r].step([shards[r]])
        return self.flat
