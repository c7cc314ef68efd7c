"""Per-op forward/backward of dtrain's autograd ops, restated as functions.

Each pair mirrors one op closure of dtrain/autograd.py with the identical NumPy
expressions, so dtype promotion (including NumPy 2's float64 promotion inside
causal attention for float32 inputs, caused by the np.float64 `scale`) and
rounding match dtrain. Test infrastructure only.
"""
from __future__ import annotations

import numpy as np


def unbroadcast(g: np.ndarray, shape: tuple) -> np.ndarray:
    """dtrain/autograd.py:29-36: sum g over the axes broadcast from `shape`."""
    while g.ndim > len(shape):
        g = g.sum(axis=0)
    for i, s in enumerate(shape):
        if s == 1 and g.shape[i] != 1:
            g = g.sum(axis=i, keepdims=True)
    return g


# ------------------------------------------------------------- elementwise
def add_bwd(g, a_shape, b_shape):
    """dtrain/autograd.py:76-84."""
    return unbroadcast(g, a_shape), unbroadcast(g, b_shape)


def mul_bwd(g, a, b):
    """dtrain/autograd.py:92-98."""
    return unbroadcast(g * b, a.shape), unbroadcast(g * a, b.shape)


def matmul_bwd(g, a, b):
    """dtrain/autograd.py:102-109: dA = g @ B^T, dB = A^T @ g, then unbroadcast."""
    ga = g @ np.swapaxes(b, -1, -2)
    gb = np.swapaxes(a, -1, -2) @ g
    return unbroadcast(ga, a.shape), unbroadcast(gb, b.shape)


def sum_bwd(g, a_shape, axis=None, keepdims=False):
    """dtrain/autograd.py:111-117."""
    if axis is not None and not keepdims:
        g = np.expand_dims(g, axis)
    return np.broadcast_to(g, a_shape).copy()


def gelu_fwd(x):
    """dtrain/autograd.py:133-139 (tanh approximation). Returns (y, t, c)."""
    c = np.sqrt(2.0 / np.pi).astype(x.dtype)
    u = c * (x + 0.044715 * x ** 3)
    t = np.tanh(u)
    y = 0.5 * x * (1.0 + t)
    return y, t, c


def gelu_bwd(g, x, t, c):
    """dtrain/autograd.py:141-143."""
    du = c * (1.0 + 3 * 0.044715 * x ** 2)
    return g * (0.5 * (1.0 + t) + 0.5 * x * (1.0 - t * t) * du)


def relu_fwd(x):
    """dtrain/autograd.py:146-148."""
    m = x > 0
    return x * m, m


def relu_bwd(g, m):
    return g * m


# ---------------------------------------------------------------- embedding
def embedding_fwd(w, idx):
    """dtrain/autograd.py:199-204 (forward gather)."""
    return w[idx]


def embedding_bwd(g, w_shape, w_dtype, idx):
    """dtrain/autograd.py:200-203: zeros, then sequential scatter-add (np.add.at)."""
    gw = np.zeros(w_shape, w_dtype)
    np.add.at(gw, idx.reshape(-1), g.reshape(-1, w_shape[1]))
    return gw


# ---------------------------------------------------------------- layer norm
def layer_norm_fwd(x, w, b, eps=1e-5):
    """dtrain/autograd.py:207-214. Returns (y, (xh, rstd))."""
    mu = x.mean(-1, keepdims=True)
    xc = x - mu
    var = (xc * xc).mean(-1, keepdims=True)
    rstd = 1.0 / np.sqrt(var + eps)
    xh = xc * rstd
    y = xh * w + b
    return y, (xh, rstd, mu)


def layer_norm_bwd(g, cache, w):
    """dtrain/autograd.py:216-222: (gx, gw, gb)."""
    xh, rstd, _ = cache
    n = xh.shape[-1]
    gxh = g * w
    gx = rstd * (gxh - gxh.mean(-1, keepdims=True) - xh * (gxh * xh).mean(-1, keepdims=True))
    gw = (g * xh).reshape(-1, n).sum(0)
    gb = g.reshape(-1, n).sum(0)
    return gx, gw, gb


# ----------------------------------------------------------------- attention
def attention_fwd(q, k, v):
    """dtrain/autograd.py:226-238 for (B, H, T, D) inputs.

    Returns (out, p, scale). `scale` is an np.float64 scalar, so for float32
    inputs s, p and the product p @ v are float64 under NumPy 2 (promotion by a
    non-weak scalar); `out` is cast back to q.dtype as dtrain does (:247).
    """
    d = q.shape[-1]
    T = q.shape[-2]
    scale = 1.0 / np.sqrt(d)
    s = (q @ np.swapaxes(k, -1, -2)) * scale
    mask = np.triu(np.ones((T, T), dtype=bool), 1)
    s = np.where(mask, -np.inf, s)
    s = s - s.max(-1, keepdims=True)
    p = np.exp(s)
    p /= p.sum(-1, keepdims=True)
    out = p @ v
    return out.astype(q.dtype, copy=False), p, scale


def attention_bwd(g, q, k, v, p, scale):
    """dtrain/autograd.py:240-246: (gq, gk, gv), in the promoted dtype."""
    gv = np.swapaxes(p, -1, -2) @ g
    gp = g @ np.swapaxes(v, -1, -2)
    gs = p * (gp - (gp * p).sum(-1, keepdims=True))
    gs *= scale
    gq = gs @ k
    gk = np.swapaxes(gs, -1, -2) @ q
    return gq, gk, gv


def softmax_bwd(p, dp):
    """Row softmax backward as used inside dtrain/autograd.py:242 (without the
    1/sqrt(d) factor): dS = P * (dP - rowsum(dP * P))."""
    return p * (dp - (dp * p).sum(-1, keepdims=True))


def row_stats(q, k):
    """Row max and row sum of exp of the masked, scaled scores (the statistics
    a flash-style forward saves), in the promoted dtype of attention_fwd."""
    d = q.shape[-1]
    T = q.shape[-2]
    scale = 1.0 / np.sqrt(d)
    s = (q @ np.swapaxes(k, -1, -2)) * scale
    s = np.where(np.triu(np.ones((T, T), dtype=bool), 1), -np.inf, s)
    m = s.max(-1)
    l = np.exp(s - m[..., None]).sum(-1)
    return m, l


# ------------------------------------------------------------- cross entropy
def cross_entropy_fwd(z, targets):
    """dtrain/autograd.py:250-260. Returns (loss 0-d array, (e, s))."""
    zmax = z.max(-1, keepdims=True)
    e = np.exp(z - zmax)
    s = e.sum(-1, keepdims=True)
    logp = (z - zmax) - np.log(s)
    flat = logp.reshape(-1, z.shape[-1])
    t = targets.reshape(-1)
    n = t.shape[0]
    loss = -flat[np.arange(n), t].mean()
    return np.asarray(loss, dtype=z.dtype), (e, s)


def cross_entropy_bwd(g, z, targets, cache):
    """dtrain/autograd.py:262-265."""
    e, s = cache
    t = targets.reshape(-1)
    n = t.shape[0]
    p = (e / s).reshape(-1, z.shape[-1]).copy()
    p[np.arange(n), t] -= 1.0
    return (p * (g / n)).reshape(z.shape).astype(z.dtype, copy=False)
