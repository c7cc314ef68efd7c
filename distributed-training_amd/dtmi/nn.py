"""Modules with dtrain's API (dtrain/nn.py): Module, Linear, LayerNorm, GPTConfig,
Block, GPT.

Same parameter order (attribute definition order, depth first), same names,
same initialisation (one NumPy default_rng(seed), same draw order and std per
tensor, float64 draws cast to the model dtype), so a dtmi GPT starts from the
very values a dtrain GPT of the same config and seed holds. After construction
GPT packs every parameter into one contiguous device buffer in that order
(`GPT.flat`); each parameter's `.data` is a view into it.

Ops are fused relative to dtrain's graph without changing the arithmetic:
Linear runs x @ w + b as one GEMM with the bias added in its epilogue (the add
node's backward becomes the GEMM's column-sum); the residual adds of
Block.forward happen in the epilogue of the GEMM that produces the branch;
the MLP's GELU and its backward run in the epilogues of the fc and out GEMMs;
and the attention block reads q, k, v straight out of the qkv projection and
writes its output in [B, T, C] order, so the reshape / transpose / split of
Block.forward (nn.py:100-103) cost no copies and the backward writes d(qkv)
in place.
"""
from __future__ import annotations

import weakref
from dataclasses import dataclass

import numpy as np

from . import device as dev
from . import kernels as K
from .autograd import Indices, Tensor, _contig, as_indices, cross_entropy, embedding, grad_out, layer_norm


class Module:
    def parameters(self):
        """All parameters in a deterministic order (attribute definition order, depth-first)."""
        out, seen = [], set()

        def walk(m):
            for v in m.__dict__.values():
                if isinstance(v, Tensor) and v.requires_grad and id(v) not in seen:
                    seen.add(id(v))
                    out.append(v)
                elif isinstance(v, Module):
                    walk(v)
                elif isinstance(v, (list, tuple)):
                    for x in v:
                        if isinstance(x, Module):
                            walk(x)
        walk(self)
        return out

    def named_parameters(self):
        names = {}

        def walk(m, prefix):
            for k, v in m.__dict__.items():
                if isinstance(v, Tensor) and v.requires_grad:
                    names.setdefault(id(v), prefix + k)
                elif isinstance(v, Module):
                    walk(v, prefix + k + ".")
                elif isinstance(v, (list, tuple)):
                    for i, x in enumerate(v):
                        if isinstance(x, Module):
                            walk(x, f"{prefix}{k}.{i}.")
        walk(self, "")
        return [(names[id(p)], p) for p in self.parameters()]

    def zero_grad(self):
        for p in self.parameters():
            p.grad = None

    def __call__(self, *a, **k):
        return self.forward(*a, **k)


def param(arr, name=None):
    return Tensor(arr, requires_grad=True, name=name)


# rowsum(dO * O) of an attention backward, formed by the projection's input-
# gradient GEMM while it produces dO (linear -> qkv_attention): keyed by that
# gradient array, so the attention backward uses it only when the gradient it
# receives is exactly that array (not a sum with another path's gradient)
_ROWSUMS: "weakref.WeakKeyDictionary" = weakref.WeakKeyDictionary()


def _with_ln(X2, W, b, R2, ln: "LayerNorm | None", lead):
    """y = residual + (x @ w + b) as [*lead, N]; with `ln`, the kernel also
    computes ln(y), returned as the (w, b, eps, y, mean, rstd) that
    layer_norm(y, w, b) takes instead of recomputing it."""
    N = W.shape[1]
    if ln is None:
        out, _ = K.linear_fwd_fused(X2, W, b, residual=R2)
        return out.reshape(*lead, N), None
    out, h, mean, rstd = K.linear_fwd_ln(X2, W, b, R2, _contig(ln.w.data), _contig(ln.b.data))
    return out.reshape(*lead, N), (ln.w, ln.b, 1e-5, h.reshape(*lead, N), mean, rstd)


def linear(x: Tensor, w: Tensor, b: Tensor | None, residual: Tensor | None = None,
           ln: "LayerNorm | None" = None) -> Tensor:
    """y = x @ w (+ b) for x [..., K], w [K, N], b [N]: one GEMM, bias fused.
    With `residual` (same shape as y): y = residual + (x @ w + b), the add
    fused into the same epilogue; its gradient passes straight through. With
    `ln`, the LayerNorm that reads y next (ln(y)) is computed in the same
    pass over y's rows."""
    X = _contig(x.data)
    lead = X.shape[:-1]
    X2 = X.reshape(-1, X.shape[-1])
    W = w.data
    R2 = _contig(residual.data).reshape(-1, W.shape[1]) if residual is not None else None
    y, pre = _with_ln(X2, W, b.data if b is not None else None, R2, ln, lead)

    def bw(g):
        g2 = _contig(g).reshape(-1, W.shape[1])
        # x is an attention output [B, T, H * 64]: dx is its dO, and the same
        # pass forms the attention backward's rowsum(dO * O)
        rs = None
        if x._rowdot is not None and x.requires_grad:
            rs = dev.empty((X.shape[0] * x._rowdot * X.shape[1],), X.dtype)
        # x is a LayerNorm output: its backward adds dx's split-K partials
        # itself, as many as it takes for this row width (float32 rows of 768:
        # four, which the vocabulary head's dX splits into)
        parts = K.ln_fusable_parts(X.dtype, X.shape[-1]) if LN_SPLIT_SUM and x._ln_out and rs is None else 0
        dx, dw, db = K.linear_bwd(X2, W, g2, need_dx=x.requires_grad, need_db=b is not None, dw_out=grad_out(w),
                                  db_out=grad_out(b) if b is not None else None, rowdot=rs,
                                  rowdot_t=X.shape[1] if rs is not None else 1, dx_parts=parts)
        out = [_shaped(dx, X.shape), dw]
        if rs is not None:
            _ROWSUMS[out[0]] = rs
        if b is not None:
            out.append(db)
        if residual is not None:
            out.append(g)
        return tuple(out)
    parents = [x, w] + ([b] if b is not None else []) + ([residual] if residual is not None else [])
    t = Tensor._make(y, tuple(parents), bw)
    t._ln_pre = pre
    return t


# The qkv and fc products read LayerNorm outputs: their input gradient goes
# to the LayerNorm backward as split-K partials (kernels.SplitSum) when the
# product is split in two, and that backward adds them while it loads its
# rows (the same bits as summing first). False sums them in a pass of their own.
LN_SPLIT_SUM = True


def _shaped(dx, shape):
    """dx (an array or a kernels.SplitSum, or None) as a gradient of `shape`."""
    if dx is None:
        return None
    if isinstance(dx, K.SplitSum):
        return K.SplitSum(dx.parts, dx.n, shape)
    return dx.reshape(shape)


def mlp(x: Tensor, fc: "Linear", out: "Linear", residual: Tensor, ln: "LayerNorm | None" = None) -> Tensor:
    """residual + out(gelu(fc(x))), Block's MLP branch (dtrain/nn.py:105) as two
    GEMMs: the fc GEMM's epilogue adds the bias and also writes gelu of the
    result, the out GEMM's epilogue adds bias and residual; in the backward
    the out layer's input-gradient GEMM applies the GELU backward in its
    epilogue (dh = gelu'(h) * (g @ W_out^T)). Same operations, same order."""
    X = _contig(x.data)
    lead = X.shape[:-1]
    X2 = X.reshape(-1, X.shape[-1])
    Wf, Wo = fc.w.data, out.w.data
    bf, bo = fc.b, out.b
    h, act = K.linear_fwd_fused(X2, Wf, bf.data if bf is not None else None, gelu=True)
    R2 = _contig(residual.data).reshape(-1, Wo.shape[1])
    y, pre = _with_ln(act, Wo, bo.data if bo is not None else None, R2, ln, lead)

    def bw(g):
        g2 = _contig(g).reshape(-1, Wo.shape[1])
        dh, dwo, dbo = K.linear_bwd(act, Wo, g2, need_dx=True, need_db=bo is not None, dw_out=grad_out(out.w),
                                    db_out=grad_out(bo) if bo is not None else None, gelu_pre=h)
        dx, dwf, dbf = K.linear_bwd(X2, Wf, dh, need_dx=x.requires_grad, need_db=bf is not None,
                                    dw_out=grad_out(fc.w), db_out=grad_out(bf) if bf is not None else None,
                                    dx_parts=2 if LN_SPLIT_SUM and x._ln_out else 0)
        res = [_shaped(dx, X.shape), dwf]
        if bf is not None:
            res.append(dbf)
        res.append(dwo)
        if bo is not None:
            res.append(dbo)
        res.append(g)
        return tuple(res)
    parents = [x, fc.w] + ([bf] if bf is not None else []) + [out.w] + ([bo] if bo is not None else []) + [residual]
    t = Tensor._make(y, tuple(parents), bw)
    t._ln_pre = pre
    return t


def qkv_attention(qkv: Tensor, heads: int) -> Tensor:
    """Causal self-attention of dtrain's Block (nn.py:100-103) on the fused
    projection qkv [B, T, 3C]: returns the merged heads [B, T, C]."""
    B, T, C3 = qkv.shape
    C = C3 // 3
    D = C // heads
    src = _contig(qkv.data)
    t5 = src.reshape(B, T, 3, heads, D).transpose(2, 0, 3, 1, 4)  # [3, B, H, T, D] view
    out = dev.empty((B, T, C), qkv.dtype)
    _, rmax, rsum = K.attn_fwd(t5[0], t5[1], t5[2], out=out.reshape(B, T, heads, D).transpose(0, 2, 1, 3))

    def bw(g):
        drow = _ROWSUMS.pop(g, None)
        gq = dev.empty((B, T, C3), qkv.dtype)
        d5 = gq.reshape(B, T, 3, heads, D).transpose(2, 0, 3, 1, 4)
        gv = _contig(g).reshape(B, T, heads, D).transpose(0, 2, 1, 3)
        o = out.reshape(B, T, heads, D).transpose(0, 2, 1, 3)
        K.attn_bwd(t5[0], t5[1], t5[2], o, gv, rmax, rsum, dq=d5[0], dk=d5[1], dv=d5[2], drow=drow)
        return (gq,)
    t = Tensor._make(out, (qkv,), bw)
    if D == 64 and qkv.dtype == np.float32:
        t._rowdot = heads  # its gradient's producer may form rowsum(dO * O) per head
    return t


class Linear(Module):
    def __init__(self, nin, nout, rng, dtype=np.float32, bias=True, std=0.02):
        self.w = param((rng.standard_normal((nin, nout)) * std).astype(dtype))
        self.b = param(np.zeros(nout, dtype)) if bias else None

    def forward(self, x):
        return linear(x, self.w, self.b)


class LayerNorm(Module):
    def __init__(self, n, dtype=np.float32):
        self.w = param(np.ones(n, dtype))
        self.b = param(np.zeros(n, dtype))

    def forward(self, x):
        return layer_norm(x, self.w, self.b)


@dataclass
class GPTConfig:
    vocab: int = 65
    ctx: int = 64
    dim: int = 128
    heads: int = 4
    layers: int = 4
    dtype: str = "float32"


class Block(Module):
    def __init__(self, c: GPTConfig, rng):
        dt = np.dtype(c.dtype)
        self.c = c
        self.ln1 = LayerNorm(c.dim, dt)
        self.qkv = Linear(c.dim, 3 * c.dim, rng, dt)
        self.proj = Linear(c.dim, c.dim, rng, dt, std=0.02 / np.sqrt(2 * c.layers))
        self.ln2 = LayerNorm(c.dim, dt)
        self.fc = Linear(c.dim, 4 * c.dim, rng, dt)
        self.out = Linear(4 * c.dim, c.dim, rng, dt, std=0.02 / np.sqrt(2 * c.layers))

    def forward(self, x, next_ln: "LayerNorm | None" = None):
        """dtrain/nn.py:98-105. `next_ln` is the LayerNorm that reads this
        block's output (the next block's ln1, or the model's final ln): the
        output GEMM computes it in the same pass over the rows, as the proj
        GEMM does for ln2."""
        a = qkv_attention(self.qkv(self.ln1(x)), self.c.heads)
        x = linear(a, self.proj.w, self.proj.b, residual=x, ln=self.ln2)  # x + self.proj(a)
        return mlp(self.ln2(x), self.fc, self.out, residual=x, ln=next_ln)  # x + self.out(self.fc(self.ln2(x)).gelu())


class GPT(Module):
    def __init__(self, c: GPTConfig, seed=0):
        rng = np.random.default_rng(seed)
        dt = np.dtype(c.dtype)
        self.c = c
        self.tok = param((rng.standard_normal((c.vocab, c.dim)) * 0.02).astype(dt))
        self.pos = param((rng.standard_normal((c.ctx, c.dim)) * 0.01).astype(dt))
        self.blocks = [Block(c, rng) for _ in range(c.layers)]
        self.ln = LayerNorm(c.dim, dt)
        self.head = Linear(c.dim, c.vocab, rng, dt, bias=False)
        self._pack()

    def _pack(self):
        """Move every parameter into one contiguous device buffer (forward order)."""
        params = self.parameters()
        n = sum(p.data.size for p in params)
        flat = dev.empty((n,), params[0].dtype)
        off = 0
        for p in params:
            k = p.data.size
            view = flat[off:off + k].reshape(p.data.shape)
            K.copy_into(view, p.data)
            p.data = view
            off += k
        self.flat = flat

    def load_numpy(self, arrays: dict):
        """Set parameters from host arrays keyed by name (e.g. a dtrain state)."""
        for name, p in self.named_parameters():
            a = np.asarray(arrays[name], dtype=p.dtype)
            if a.shape != p.shape:
                raise ValueError(f"{name}: shape {a.shape} != {p.shape}")
            p.data.assign(a)

    def state_numpy(self) -> dict:
        return {name: p.numpy() for name, p in self.named_parameters()}

    def _positions(self, T: int) -> Indices:
        cache = self.__dict__.setdefault("_pos_ids", {})
        if T not in cache:
            cache[T] = Indices(np.arange(T))
        return cache[T]

    def forward(self, idx, targets=None):
        """idx, targets: host integer arrays or Indices (uploaded once)."""
        idx = as_indices(idx)
        B, T = idx.shape
        x = embedding(self.tok, idx) + embedding(self.pos, self._positions(T))
        for i, b in enumerate(self.blocks):
            x = b(x, next_ln=self.blocks[i + 1].ln1 if i + 1 < len(self.blocks) else self.ln)
        logits = self.head(self.ln(x))
        if targets is None:
            return logits
        return logits, cross_entropy(logits, targets)
