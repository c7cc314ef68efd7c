"""One training step of dtrain (dtrain/train.py:128-159) on one GPU.

`step_single`: `--mode single` with `--emulate-world W` (each virtual rank's
loss scaled by 1/(accum*W), leaf gradients accumulate; train.py:130-145),
then the global-norm clip and AdamW.

`step_ddp`: `--mode ddp` with W simulated replicas (each replica's loss scaled
by 1/accum; gradients through DDP buckets and the fixed-order average), then
clip and AdamW.

`step_zero`: `--mode zero` with W simulated replicas and ZeroAdamW.

The global norm, the clip factor and the optimizer all stay on the device (no
host round trip inside a step); the returned loss and gradient norm are device
scalars that `float()` reads back when they are needed. `lr_at` is dtrain's
warm-up + cosine schedule (train.py:63-69).
"""
from __future__ import annotations

import numpy as np

from .optim import clip_scale_device, grad_sq_norm


def lr_at(step: int, lr: float, warmup: int, steps: int) -> float:
    """dtrain/train.py:63-69."""
    if warmup and step < warmup:
        return lr * (step + 1) / warmup
    if not warmup:
        return lr
    t = (step - warmup) / max(1, steps - warmup)
    return lr * (0.1 + 0.9 * 0.5 * (1 + np.cos(np.pi * min(1.0, t))))


class StepResult:
    def __init__(self, losses, n_micro, world, norm, scale=1.0):
        self._losses, self._n_micro, self._world, self._norm = losses, n_micro, world, norm
        self._scale = scale

    @property
    def loss(self) -> float:
        """Mean loss as dtrain logs it (train.py:145, 160-163)."""
        per_rank = {}
        for r, l in self._losses:
            per_rank[r] = per_rank.get(r, 0.0) + float(l.numpy()) / self._n_micro
        total = 0.0
        for r in sorted(per_rank):
            total += per_rank[r]
        return total / self._world if self._world > 1 else total

    @property
    def grad_norm(self) -> float:
        return float(self._norm.numpy()[0])

    @property
    def clip_scale(self) -> float:
        """The factor the gradients were multiplied by inside AdamW."""
        s = self._scale
        return float(s.numpy()[0]) if hasattr(s, "numpy") else float(s)


def _clip(sq, clip):
    if clip:
        return clip_scale_device(sq, clip)
    s, n = clip_scale_device(sq, float("inf"))
    return 1.0, n


def step_single(model, opt, batches, clip=1.0, accum=1):
    """batches[vr][micro] = (x, y) host token arrays, one list per virtual rank."""
    params = model.parameters()
    model.zero_grad()
    vworlds = len(batches)
    n_micro = accum * vworlds
    losses = []
    for micro in range(accum):
        for vr in range(vworlds):
            x, y = batches[vr][micro]
            _, loss = model(x, y)
            (loss * (1.0 / n_micro)).backward()
            losses.append((0, loss.data))
    sq = grad_sq_norm([p.grad for p in params])
    s, norm = _clip(sq, clip)
    opt.step([p.grad for p in params], grad_scale=s)
    return StepResult(losses, n_micro, 1, norm, s)


def step_ddp(model, ddp, opt, batches, clip=1.0, accum=1):
    """batches[r][micro] = (x, y) for simulated rank r."""
    pg = ddp.pg
    params = model.parameters()
    losses = []
    for r in range(pg.world):
        with pg.replica(r):
            model.zero_grad()
            for micro in range(accum):
                x, y = batches[r][micro]
                _, loss = model(x, y)
                scaled = loss * (1.0 / accum)
                if micro < accum - 1:
                    with ddp.no_sync():
                        scaled.backward()
                else:
                    scaled.backward()
                losses.append((r, loss.data))
    ddp.finish()
    s, norm = _clip(ddp.grad_sq, clip)
    opt.step([p.grad for p in params], grad_scale=s)
    return StepResult(losses, accum, pg.world, norm, s)


def step_zero(model, zero, batches, accum=1):
    pg = zero.pg
    losses = []
    for r in range(pg.world):
        with pg.replica(r):
            model.zero_grad()
            for micro in range(accum):
                x, y = batches[r][micro]
                _, loss = model(x, y)
                (loss * (1.0 / accum)).backward()
                losses.append((r, loss.data))
    zero.step()
    return StepResult(losses, accum, pg.world, zero.last_grad_norm_device)
