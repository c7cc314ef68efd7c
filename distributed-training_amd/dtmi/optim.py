"""AdamW over device arrays with dtrain's API (dtrain/optim.py).

`AdamW(params, lr, betas, eps, weight_decay)` keeps m and v in one flat device
buffer (a view per parameter) and updates every (p, g, m, v) of a step in one
fused multi-tensor kernel: read p, g, m, v once, write p, m, v once. The
update is dtrain's operation order (optim.py:28-33) in IEEE arithmetic without
FMA contraction, so float64 results are bit-identical to dtrain's NumPy step.

`step(grads, grad_scale=...)` also takes the clip factor, so the
`opt.step([p.grad * s ...])` of dtrain/train.py:159 costs no extra pass over
the gradients; grad_scale may be a Python float or a 1-element float64 device
array (the factor computed on the device by dtmi_clip_scale).
"""
from __future__ import annotations

import numpy as np

from . import device as dev
from . import kernels as K
from .device import DeviceArray


def _one_run(arrays):
    """A 1-D view covering `arrays` when they are contiguous and lie back to
    back in one allocation (in list order), else None."""
    if not arrays or any(a is None or not a.is_contiguous for a in arrays):
        return None
    a0 = arrays[0]
    end = a0.offset + a0.nbytes
    for a in arrays[1:]:
        if a.block is not a0.block or a.offset != end or a.dtype != a0.dtype:
            return None
        end += a.nbytes
    return DeviceArray(a0.block, ((end - a0.offset) // a0.itemsize,), a0.dtype, a0.offset)


class AdamW:
    def __init__(self, params, lr=3e-4, betas=(0.9, 0.95), eps=1e-8, weight_decay=0.1):
        self.params = list(params)  # DeviceArrays, updated in place
        self.lr, self.b1, self.b2, self.eps, self.wd = lr, betas[0], betas[1], eps, weight_decay
        n = sum(p.size for p in self.params)
        dt = self.params[0].dtype if self.params else np.float32
        self._mflat = dev.zeros((max(n, 1),), dt)
        self._vflat = dev.zeros((max(n, 1),), dt)
        self.m, self.v = [], []
        off = 0
        for p in self.params:
            k = p.size
            self.m.append(self._mflat[off:off + k].reshape(p.shape))
            self.v.append(self._vflat[off:off + k].reshape(p.shape))
            off += k
        self.t = 0

    def step(self, grads, grad_scale=1.0):
        """dtrain/optim.py:21-33. grads: DeviceArray or None per parameter."""
        self.t += 1
        b1t = 1 - self.b1 ** self.t
        b2t = 1 - self.b2 ** self.t
        gs_dev = grad_scale if isinstance(grad_scale, DeviceArray) else None
        gs = 1.0 if gs_dev is not None else float(grad_scale)
        grads = list(grads)
        P, G = _one_run(self.params), _one_run(grads)
        if P is not None and G is not None:
            # parameters and gradients are each one contiguous run (e.g. a
            # packed model and DDP's averaged gradients): one flat launch
            n = P.size
            K.adamw(P, G, self._mflat[:n], self._vflat[:n], self.lr, self.b1, self.b2, self.eps, self.wd,
                    b1t, b2t, gscale=gs, gscale_dev=gs_dev)
            return
        gl = [None if g is None else (g if g.is_contiguous else g.contiguous()) for g in grads]
        K.adamw_multi(self.params, gl, self.m, self.v, self.lr, self.b1, self.b2, self.eps, self.wd, b1t, b2t,
                      gscale=gs, gscale_dev=gs_dev)

    def state_bytes(self):
        return sum(a.nbytes for a in self.m) + sum(a.nbytes for a in self.v)

    def state_dict(self):
        return {"t": self.t, "m": [a.numpy() for a in self.m], "v": [a.numpy() for a in self.v]}

    def load_state_dict(self, s):
        self.t = int(s["t"])
        for dst, src in zip(self.m, s["m"]):
            dst.assign(src)
        for dst, src in zip(self.v, s["v"]):
            dst.assign(src)


def clip_scale(total_sq_norm: float, max_norm: float) -> float:
    """dtrain/optim.py:49-52."""
    n = float(np.sqrt(total_sq_norm))
    return 1.0 if n <= max_norm or n == 0 else max_norm / (n + 1e-6)


def grad_sq_norm(grads, out: DeviceArray | None = None) -> DeviceArray:
    """Global float64 sum of squares of the gradients (dtrain/train.py:155-156),
    deterministic, left on the device as a 1-element float64 array."""
    out = out if out is not None else dev.empty((1,), np.float64)
    K.sumsq([g if g.is_contiguous else g.contiguous() for g in grads if g is not None], out)
    return out


def clip_scale_device(sq: DeviceArray, max_norm: float):
    """clip_scale computed on the device from a device sum of squares: returns
    (scale, norm) as 1-element float64 device arrays (no host round trip)."""
    s = dev.empty((1,), np.float64)
    n = dev.empty((1,), np.float64)
    K.clip_scale(sq, max_norm, s, n)
    return s, n
