"""dtrain's char-GPT restated as explicit forward and backward passes.

dtrain builds the graph with its autograd engine (dtrain/nn.py:87-139) and
differentiates it with Tensor.backward (dtrain/autograd.py:151-195). Here the
same per-op NumPy expressions (oracle.ops) are chained by hand: forward keeps
each op's saved values, backward applies the op backward closures in reverse.
Every node of the GPT graph that receives gradient from more than one consumer
receives exactly two (residual stream) or three with disjoint support (the
q/k/v split), so the summation order of the engine cannot change any bit.

Test infrastructure only.
"""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np

from . import ops


@dataclass
class GPTConfig:
    """dtrain/nn.py:77-84."""
    vocab: int = 65
    ctx: int = 64
    dim: int = 128
    heads: int = 4
    layers: int = 4
    dtype: str = "float32"


def param_spec(c: GPTConfig):
    """Names and shapes in dtrain's parameter order (dtrain/nn.py:12-44: attribute
    definition order, depth first): tok, pos, per block ln1.{w,b}, qkv.{w,b},
    proj.{w,b}, ln2.{w,b}, fc.{w,b}, out.{w,b}; then ln.{w,b}, head.w."""
    C, V = c.dim, c.vocab
    spec = [("tok", (V, C)), ("pos", (c.ctx, C))]
    for i in range(c.layers):
        p = f"blocks.{i}."
        spec += [(p + "ln1.w", (C,)), (p + "ln1.b", (C,)),
                 (p + "qkv.w", (C, 3 * C)), (p + "qkv.b", (3 * C,)),
                 (p + "proj.w", (C, C)), (p + "proj.b", (C,)),
                 (p + "ln2.w", (C,)), (p + "ln2.b", (C,)),
                 (p + "fc.w", (C, 4 * C)), (p + "fc.b", (4 * C,)),
                 (p + "out.w", (4 * C, C)), (p + "out.b", (C,))]
    spec += [("ln.w", (C,)), ("ln.b", (C,)), ("head.w", (C, V))]
    return spec


def dtrain_init(c: GPTConfig, seed: int = 0) -> dict:
    """dtrain's GPT initialisation (dtrain/nn.py:58-61, 68-71, 87-96, 121-129):
    one default_rng(seed); draws in construction order; each matrix is a float64
    standard normal times its std, then cast; biases 0, LayerNorm w=1 b=0."""
    rng = np.random.default_rng(seed)
    dt = np.dtype(c.dtype)
    C, V, L = c.dim, c.vocab, c.layers
    out = {"tok": (rng.standard_normal((V, C)) * 0.02).astype(dt),
           "pos": (rng.standard_normal((c.ctx, C)) * 0.01).astype(dt)}
    small = 0.02 / np.sqrt(2 * L)
    for i in range(L):
        p = f"blocks.{i}."
        out[p + "ln1.w"] = np.ones(C, dt)
        out[p + "ln1.b"] = np.zeros(C, dt)
        out[p + "qkv.w"] = (rng.standard_normal((C, 3 * C)) * 0.02).astype(dt)
        out[p + "qkv.b"] = np.zeros(3 * C, dt)
        out[p + "proj.w"] = (rng.standard_normal((C, C)) * small).astype(dt)
        out[p + "proj.b"] = np.zeros(C, dt)
        out[p + "ln2.w"] = np.ones(C, dt)
        out[p + "ln2.b"] = np.zeros(C, dt)
        out[p + "fc.w"] = (rng.standard_normal((C, 4 * C)) * 0.02).astype(dt)
        out[p + "fc.b"] = np.zeros(4 * C, dt)
        out[p + "out.w"] = (rng.standard_normal((4 * C, C)) * small).astype(dt)
        out[p + "out.b"] = np.zeros(C, dt)
    out["ln.w"] = np.ones(C, dt)
    out["ln.b"] = np.zeros(C, dt)
    out["head.w"] = (rng.standard_normal((C, V)) * 0.02).astype(dt)
    return {name: out[name] for name, _ in param_spec(c)}


def synthetic_init(c: GPTConfig, seed: int = 0, std: float = 0.02) -> dict:
    """The benchmark workloads' weights: every matrix N(0, std) (float64 draw,
    then cast, in parameter order from default_rng(seed)); biases 0; LayerNorm
    w=1, b=0."""
    rng = np.random.default_rng(seed)
    dt = np.dtype(c.dtype)
    out = {}
    for name, shape in param_spec(c):
        leaf = name.rsplit(".", 1)[-1]
        if len(shape) == 2:
            out[name] = (rng.standard_normal(shape) * std).astype(dt)
        elif ".ln" in "." + name and leaf == "w":
            out[name] = np.ones(shape, dt)
        else:
            out[name] = np.zeros(shape, dt)
    return out


def synthetic_tokens(c: GPTConfig, batch: int, seed: int, replicas: int = 1):
    """Uniform token ids in [0, vocab): for each replica r, x then y, both
    (batch, ctx), from one default_rng(seed)."""
    rng = np.random.default_rng(seed)
    xs, ys = [], []
    for _ in range(replicas):
        xs.append(rng.integers(0, c.vocab, (batch, c.ctx)))
        ys.append(rng.integers(0, c.vocab, (batch, c.ctx)))
    return xs, ys


# ------------------------------------------------------------------ model
def _linear_fwd(x, w, b):
    """dtrain/nn.py:63-65: x @ w (+ b)."""
    y = x @ w
    return y + b if b is not None else y


def _linear_bwd(g, x, w, has_bias):
    """Backward of `x @ w + b`: the add node (autograd.py:80-82) then the matmul
    node (autograd.py:105-108)."""
    gb = ops.unbroadcast(g, (w.shape[1],)) if has_bias else None
    gx, gw = ops.matmul_bwd(g, x, w)
    return gx, gw, gb


def forward(P: dict, c: GPTConfig, idx: np.ndarray, targets: np.ndarray):
    """dtrain/nn.py:131-139 and Block.forward (nn.py:98-105). Returns
    (logits, loss, tape) where tape holds what backward needs."""
    B, T = idx.shape
    C, H = c.dim, c.heads
    D = C // H
    tape = {"idx": idx, "targets": targets, "blocks": []}
    x = ops.embedding_fwd(P["tok"], idx) + ops.embedding_fwd(P["pos"], np.arange(T))
    for i in range(c.layers):
        p = f"blocks.{i}."
        bt = {}
        bt["x_in"] = x
        h1, bt["ln1"] = ops.layer_norm_fwd(x, P[p + "ln1.w"], P[p + "ln1.b"])
        bt["h1"] = h1
        qkv = _linear_fwd(h1, P[p + "qkv.w"], P[p + "qkv.b"])
        t5 = qkv.reshape(B, T, 3, H, D).transpose(2, 0, 3, 1, 4)
        q, k, v = t5[0], t5[1], t5[2]
        bt["qkv_dtype"] = qkv.dtype
        a, pr, scale = ops.attention_fwd(q, k, v)
        bt["att"] = (q, k, v, pr, scale)
        a2 = a.transpose(0, 2, 1, 3).reshape(B, T, C)
        bt["a2"] = a2
        x = x + _linear_fwd(a2, P[p + "proj.w"], P[p + "proj.b"])
        bt["x_mid"] = x
        h2, bt["ln2"] = ops.layer_norm_fwd(x, P[p + "ln2.w"], P[p + "ln2.b"])
        bt["h2"] = h2
        f = _linear_fwd(h2, P[p + "fc.w"], P[p + "fc.b"])
        gl, t, cc = ops.gelu_fwd(f)
        bt["gelu"] = (f, t, cc)
        bt["gl"] = gl
        x = x + _linear_fwd(gl, P[p + "out.w"], P[p + "out.b"])
        tape["blocks"].append(bt)
    hf, tape["lnf"] = ops.layer_norm_fwd(x, P["ln.w"], P["ln.b"])
    tape["hf"] = hf
    logits = _linear_fwd(hf, P["head.w"], None)
    loss, tape["ce"] = ops.cross_entropy_fwd(logits, targets)
    tape["logits"] = logits
    return logits, loss, tape


def backward(P: dict, c: GPTConfig, tape: dict, loss_scale: float = 1.0) -> dict:
    """Gradients of `loss * loss_scale` (dtrain/train.py:138) w.r.t. every
    parameter, following Tensor.backward's reverse order of the GPT graph."""
    dt = np.dtype(c.dtype)
    idx, targets = tape["idx"], tape["targets"]
    B, T = idx.shape
    C, H = c.dim, c.heads
    D = C // H
    G = {}
    # seed: ones_like(scaled) then the `loss * (1/n)` node (autograd.py:92-98)
    g_scaled = np.ones((), dt)
    g_loss = ops.unbroadcast(g_scaled * np.asarray(loss_scale, dtype=dt), ())
    glogits = ops.cross_entropy_bwd(g_loss, tape["logits"], targets, tape["ce"])
    ghf, G["head.w"], _ = _linear_bwd(glogits, tape["hf"], P["head.w"], False)
    gx, G["ln.w"], G["ln.b"] = ops.layer_norm_bwd(ghf, tape["lnf"], P["ln.w"])
    for i in reversed(range(c.layers)):
        p = f"blocks.{i}."
        bt = tape["blocks"][i]
        # x_out = x_mid + out(gelu(fc(ln2(x_mid))))
        ggl, G[p + "out.w"], G[p + "out.b"] = _linear_bwd(gx, bt["gl"], P[p + "out.w"], True)
        f, t, cc = bt["gelu"]
        gf = ops.gelu_bwd(ggl, f, t, cc)
        gh2, G[p + "fc.w"], G[p + "fc.b"] = _linear_bwd(gf, bt["h2"], P[p + "fc.w"], True)
        gxm_ln, G[p + "ln2.w"], G[p + "ln2.b"] = ops.layer_norm_bwd(gh2, bt["ln2"], P[p + "ln2.w"])
        gxm = gx + gxm_ln
        # x_mid = x_in + proj(a2)
        ga2, G[p + "proj.w"], G[p + "proj.b"] = _linear_bwd(gxm, bt["a2"], P[p + "proj.w"], True)
        ga = ga2.reshape(B, T, H, D).transpose(0, 2, 1, 3)
        q, k, v, pr, scale = bt["att"]
        gq, gk, gv = ops.attention_bwd(ga, q, k, v, pr, scale)
        # _split3 backward (nn.py:108-117): each grad lands in its slot of a
        # zeros_like(qkv-transposed) array of the qkv dtype (casts float64
        # attention grads back to float32 for a float32 model)
        full = np.zeros((3, B, H, T, D), bt["qkv_dtype"])
        full[0] = gq
        full[1] = gk
        full[2] = gv
        gqkv = full.transpose(1, 3, 0, 2, 4).reshape(B, T, 3 * C)
        gh1, G[p + "qkv.w"], G[p + "qkv.b"] = _linear_bwd(gqkv, bt["h1"], P[p + "qkv.w"], True)
        gxi_ln, G[p + "ln1.w"], G[p + "ln1.b"] = ops.layer_norm_bwd(gh1, bt["ln1"], P[p + "ln1.w"])
        gx = gxm + gxi_ln
    # x0 = tok[idx] + pos[arange(T)]
    g_tok_rows, g_pos_rows = ops.add_bwd(gx, (B, T, C), (T, C))
    G["tok"] = ops.embedding_bwd(g_tok_rows, P["tok"].shape, P["tok"].dtype, idx)
    G["pos"] = ops.embedding_bwd(g_pos_rows, P["pos"].shape, P["pos"].dtype, np.arange(T))
    return {name: G[name] for name, _ in param_spec(c)}


def loss_and_grads(P, c, idx, targets, loss_scale=1.0):
    _, loss, tape = forward(P, c, idx, targets)
    return loss, backward(P, c, tape, loss_scale)
