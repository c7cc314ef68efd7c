"""Synthetic inputs of the benchmark workloads (host arrays, NumPy PCG64).

The parameter order is dtrain's (dtrain/nn.py:12-44: tok, pos, per block
ln1.{w,b}, qkv.{w,b}, proj.{w,b}, ln2.{w,b}, fc.{w,b}, out.{w,b}; then ln.{w,b},
head.w) and the one dtmi.nn.GPT registers. Weights: every matrix N(0, std)
drawn as float64 from one default_rng(seed) in parameter order and cast;
biases 0; LayerNorm w = 1, b = 0. Tokens: per replica x then y, each
(batch, ctx) uniform over the vocabulary from one default_rng(seed).
"""
from __future__ import annotations

import numpy as np

from .nn import GPTConfig

N_BUCKET_WORKLOAD = 124_439_808  # GPT-2-small's canonical parameter count


def param_spec(c: GPTConfig):
    """(name, shape) of every parameter in registration order."""
    C, V = c.dim, c.vocab
    spec = [("tok", (V, C)), ("pos", (c.ctx, C))]
    for i in range(c.layers):
        p = f"blocks.{i}."
        spec += [(p + "ln1.w", (C,)), (p + "ln1.b", (C,)), (p + "qkv.w", (C, 3 * C)), (p + "qkv.b", (3 * C,)),
                 (p + "proj.w", (C, C)), (p + "proj.b", (C,)), (p + "ln2.w", (C,)), (p + "ln2.b", (C,)),
                 (p + "fc.w", (C, 4 * C)), (p + "fc.b", (4 * C,)), (p + "out.w", (4 * C, C)), (p + "out.b", (C,))]
    return spec + [("ln.w", (C,)), ("ln.b", (C,)), ("head.w", (C, V))]


def synthetic_weights(c: GPTConfig, seed: int, std: float = 0.02) -> dict:
    rng = np.random.default_rng(seed)
    dt = np.dtype(c.dtype)
    out = {}
    for name, shape in param_spec(c):
        if len(shape) == 2:
            out[name] = (rng.standard_normal(shape) * std).astype(dt)
        elif ".ln" in "." + name and name.endswith(".w"):
            out[name] = np.ones(shape, dt)
        else:
            out[name] = np.zeros(shape, dt)
    return out


def synthetic_tokens(c: GPTConfig, batch: int, seed: int, replicas: int = 1):
    rng = np.random.default_rng(seed)
    xs, ys = [], []
    for _ in range(replicas):
        xs.append(rng.integers(0, c.vocab, (batch, c.ctx)))
        ys.append(rng.integers(0, c.vocab, (batch, c.ctx)))
    return xs, ys


class BucketParams:
    """The gradient-bucket workload's flat buffer of n parameters as dtrain's
    DDP would bucket it at `bucket_mb` (dtrain/ddp.py:46-56: parameters in
    reverse order, a bucket closed as soon as it holds the limit): a leading
    remainder, then n // per full-size pieces (per = the elements of one
    bucket), so the greedy rule gives one bucket per full piece and one for
    the remainder (124,439,808 float32 elements at 1 MiB: 474 full buckets of
    262,144 and one of 183,552). Each piece is a leaf Tensor viewing `flat`.
    """

    def __init__(self, flat, bucket_mb: float = 1.0):
        from .autograd import Tensor
        n = flat.size
        per = int(bucket_mb * (1 << 20)) // flat.itemsize
        rem = n % per
        sizes = ([rem] if rem else []) + [per] * (n // per)
        self.sizes = sizes
        self.ps, off = [], 0
        for k in sizes:
            self.ps.append(Tensor(flat[off:off + k], requires_grad=True))
            off += k

    def parameters(self):
        return self.ps

    def hand_over(self, ddp):
        """Every replica's gradients as they sit in DDP's replica rows: each
        parameter's slot of row r is handed to the grad-ready hook in
        reverse parameter order (the order the backward produces them), so
        the bucket averages launch as DDP.finish and the hooks issue them."""
        pg = ddp.pg
        for r in range(pg.world):
            with pg.replica(r):
                for i in reversed(range(len(self.ps))):
                    p = self.ps[i]
                    p.grad = ddp.grads.slot(r, i)
                    ddp._on_grad(p)
        ddp.finish()
