"""AdamW and the clip factor, restated from dtrain/optim.py. Test infrastructure only."""
from __future__ import annotations

import numpy as np


class AdamW:
    """dtrain/optim.py:7-46: per-array m, v; shared step count t; arrays updated
    in place with the exact in-place NumPy sequence of optim.py:28-33."""

    def __init__(self, params, lr=3e-4, betas=(0.9, 0.95), eps=1e-8, weight_decay=0.1):
        self.params = list(params)
        self.lr, self.b1, self.b2, self.eps, self.wd = lr, betas[0], betas[1], eps, weight_decay
        self.m = [np.zeros_like(p) for p in self.params]
        self.v = [np.zeros_like(p) for p in self.params]
        self.t = 0

    def step(self, grads):
        self.t += 1
        b1t = 1 - self.b1 ** self.t
        b2t = 1 - self.b2 ** self.t
        for p, g, m, v in zip(self.params, grads, self.m, self.v):
            if g is None:
                continue
            adamw_update(p, g, m, v, self.lr, self.b1, self.b2, self.eps, self.wd, b1t, b2t)

    def state_bytes(self):
        return sum(a.nbytes for a in self.m) + sum(a.nbytes for a in self.v)


def adamw_update(p, g, m, v, lr, b1, b2, eps, wd, b1t, b2t):
    """One array of dtrain/optim.py:28-33 (in place)."""
    m *= b1
    m += (1 - b1) * g
    v *= b2
    v += (1 - b2) * (g * g)
    p -= lr * (wd * p)
    p -= lr * (m / b1t) / (np.sqrt(v / b2t) + eps)


def bias_corrections(b1: float, b2: float, t: int):
    """dtrain/optim.py:22-24 with t already incremented."""
    return 1 - b1 ** t, 1 - b2 ** t


def clip_scale(total_sq_norm: float, max_norm: float) -> float:
    """dtrain/optim.py:49-52."""
    n = float(np.sqrt(total_sq_norm))
    return 1.0 if n <= max_norm or n == 0 else max_norm / (n + 1e-6)


def global_sq_norm(grads) -> float:
    """dtrain/train.py:155-156: per-array float64 dot, Python sum in array order."""
    return sum(float(np.dot(g.reshape(-1).astype(np.float64), g.reshape(-1).astype(np.float64)))
               for g in grads if g is not None)
