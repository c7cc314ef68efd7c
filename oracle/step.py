"""One training step of dtrain (dtrain/train.py:128-159), restated.

`single_step` is `--mode single` (emulate_world W: each virtual rank's loss is
scaled by 1/(accum*W) and leaf gradients accumulate, train.py:130-145).
`ddp_step` is `--mode ddp` for W ranks simulated in turn: each replica's loss
is scaled by 1/accum, gradients go through DDP's buckets and the average in
the all-reduce order of `algo` (ddp.py:84-110; "ring" is dtrain's default
--algo, "direct" sums in rank order), then the global-norm clip
(train.py:155-158) and AdamW on `p.grad * s` (train.py:159).
Test infrastructure only.
"""
from __future__ import annotations

import numpy as np

from . import model
from .ddp import ddp_average
from .optim import AdamW, clip_scale, global_sq_norm


def single_step(P, c, batches, opt: AdamW, clip=1.0, emulate_world=1, accum=1):
    """batches: list (one per virtual rank) of (x, y); with accum > 1, of accum
    (x, y) pairs each. Micro-steps outer, virtual ranks inner (train.py:132-145).
    Returns (loss, grad_norm, grads)."""
    names = list(P.keys())
    n_micro = accum * emulate_world
    grads = {k: None for k in names}
    loss_sum = 0.0
    for micro in range(accum):
        for vr in range(emulate_world):
            x, y = batches[vr] if accum == 1 else batches[vr][micro]
            loss, g = model.loss_and_grads(P, c, x, y, loss_scale=1.0 / n_micro)
            for k in names:
                grads[k] = g[k] if grads[k] is None else grads[k] + g[k]
            loss_sum += float(loss) / n_micro
    glist = [grads[k] for k in names]
    sq = global_sq_norm(glist)
    gnorm = float(np.sqrt(sq))
    s = clip_scale(sq, clip) if clip else 1.0
    opt.step([g * s if g is not None else None for g in glist])
    return loss_sum, gnorm, glist


def ddp_step(P, c, batches, opt: AdamW, clip=1.0, bucket_mb=1.0, algo="direct"):
    """batches: list (one per simulated rank) of (x, y). Returns
    (mean loss, grad_norm, averaged grads)."""
    names = list(P.keys())
    W = len(batches)
    replica_grads, losses = [], []
    for r in range(W):
        x, y = batches[r]
        loss, g = model.loss_and_grads(P, c, x, y, loss_scale=1.0)
        replica_grads.append([g[k] for k in names])
        losses.append(float(loss))
    itemsize = np.dtype(c.dtype).itemsize
    avg = ddp_average(replica_grads, itemsize, bucket_mb, algo)
    sq = global_sq_norm(avg)
    gnorm = float(np.sqrt(sq))
    s = clip_scale(sq, clip) if clip else 1.0
    opt.step([g * s if g is not None else None for g in avg])
    loss = 0.0
    for l in losses:  # the loss all-reduce, rank order, then / W (train.py:160-163)
        loss += l
    return loss / W, gnorm, avg
