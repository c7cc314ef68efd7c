"""Reverse-mode autograd over device arrays, with dtrain's Tensor API.

Mirrors dtrain/autograd.py: `Tensor(data, requires_grad, name)`, `.grad`,
`.backward(grad=None)`, `.register_grad_ready_hook(fn)`, the operators
`+ - * @`, `.sum .mean .reshape .transpose .gelu .relu`, and the functional ops
`embedding`, `layer_norm`, `causal_attention`, `cross_entropy`, `no_grad`.

Differences from dtrain are in where the numbers live, not in semantics:
`.data` and `.grad` are DeviceArrays (HBM buffers owned by libdtmi; `.numpy()`
and `np.asarray` copy to the host), and every op's forward and backward is a
libdtmi kernel launch. `backward()` is dtrain's algorithm (autograd.py:151-195):
a topological order, a reverse walk, leaf accumulation `grad = g` or
`grad + g`, and grad-ready hooks called once per leaf with its final gradient.
"""
from __future__ import annotations

import numpy as np

from . import device as dev
from . import kernels as K
from .device import DeviceArray

_grad_enabled = True


class no_grad:
    """dtrain/autograd.py:19-26."""

    def __enter__(self):
        global _grad_enabled
        self.prev, _grad_enabled = _grad_enabled, False

    def __exit__(self, *a):
        global _grad_enabled
        _grad_enabled = self.prev


def _contig(x: DeviceArray) -> DeviceArray:
    return x if x.is_contiguous else x.contiguous()


def _unbroadcast(g: DeviceArray, shape: tuple) -> DeviceArray:
    """dtrain/autograd.py:29-36: sum g over the axes broadcast from `shape`."""
    shape = tuple(shape)
    if g.shape == shape:
        return g
    lead = g.ndim - len(shape)
    if lead > 0:
        g = _contig(g)
        rest = g.shape[lead:]
        if len(rest) == 1:  # [.., N] -> [N]: deterministic two-stage column sum
            g = K.colsum(g.reshape(-1, rest[0]))
        else:
            g = K.reduce_sum(g, list(range(lead)))
    axes = [i for i, s in enumerate(shape) if s == 1 and g.shape[i] != 1]
    if axes:
        g = K.reduce_sum(g, axes, keepdims=True)
    return g


def _broadcast_to(g: DeviceArray, shape) -> DeviceArray:
    """np.broadcast_to(g, shape).copy() on the device."""
    shape = tuple(shape)
    out = dev.empty(shape, g.dtype)
    if out.size == 0:
        return out
    nd = len(shape)
    pad = nd - g.ndim
    st = [0] * pad + [0 if (s == 1 and shape[pad + i] != 1) else g.strides[i] for i, s in enumerate(g.shape)]
    view = DeviceArray(g.block, shape, g.dtype, g.offset, st)
    K.copy_into(out, view)
    return out


class Tensor:
    __slots__ = ("data", "grad", "requires_grad", "_parents", "_backward", "_hooks", "name", "grad_dest",
                 "_dest_live", "_ln_pre", "_rowdot", "_ln_out", "__weakref__")

    def __init__(self, data, requires_grad=False, _parents=(), _backward=None, name=None):
        self.data = data if isinstance(data, DeviceArray) else dev.asarray(np.asarray(data))
        self.grad = None
        self.requires_grad = requires_grad
        self._parents = _parents
        self._backward = _backward
        self._hooks = []
        self.name = name
        # Optional preallocated home for this leaf's gradient (same shape and
        # dtype), e.g. its slot in a gradient bucket: the kernel producing
        # the gradient writes straight into it, so the bucket needs no copy.
        self.grad_dest = None
        self._dest_live = None
        # A LayerNorm of this tensor computed by the kernel that produced it
        # (w, b, eps, y, mean, rstd); layer_norm(self, w, b, eps) takes it once.
        self._ln_pre = None
        self._rowdot = None
        # the output of layer_norm: the backward of the product that reads it
        # may hand its gradient over as split-K partials (kernels.SplitSum),
        # which the LayerNorm backward adds as it loads them
        self._ln_out = False

    # ------------------------------------------------------------ utilities
    @property
    def shape(self):
        return self.data.shape

    @property
    def dtype(self):
        return self.data.dtype

    def numpy(self):
        return self.data.numpy()

    def register_grad_ready_hook(self, fn):
        """fn(tensor) is called once this leaf's gradient is complete."""
        self._hooks.append(fn)

    def __repr__(self):
        return f"Tensor(shape={self.shape}, dtype={self.dtype}, requires_grad={self.requires_grad})"

    @staticmethod
    def _make(data, parents, backward):
        rg = _grad_enabled and any(p.requires_grad for p in parents)
        return Tensor(data, rg, parents if rg else (), backward if rg else None)

    def _wrap(self, o):
        return o if isinstance(o, Tensor) else Tensor(np.asarray(o, dtype=self.dtype))

    # ---------------------------------------------------------------- ops
    def __add__(self, o):
        a, b = self, self._wrap(o)

        def bw(g):
            return _unbroadcast(g, a.shape), _unbroadcast(g, b.shape)
        return Tensor._make(K.binary("add", a.data, b.data), (a, b), bw)

    __radd__ = __add__

    def __neg__(self):
        return Tensor._make(K.neg(self.data), (self,), lambda g: (K.neg(g),))

    def __sub__(self, o):
        return self + (-self._wrap(o))

    def __mul__(self, o):
        a, b = self, self._wrap(o)

        def bw(g):
            return (_unbroadcast(K.binary("mul", g, b.data), a.shape),
                    _unbroadcast(K.binary("mul", g, a.data), b.shape))
        return Tensor._make(K.binary("mul", a.data, b.data), (a, b), bw)

    __rmul__ = __mul__

    def __matmul__(self, o):
        a, b = self, o
        A, B = _contig(a.data), _contig(b.data)
        if A.ndim >= 2 and B.ndim == 2:
            lead = A.shape[:-1]
            y = K.gemm(A.reshape(-1, A.shape[-1]), B).reshape(*lead, B.shape[1])

            def bw(g):
                g2 = _contig(g).reshape(-1, B.shape[1])
                A2 = A.reshape(-1, A.shape[-1])
                ga = K.gemm(g2, B, a_kcontig=True, b_kcontig=True).reshape(A.shape)  # g @ b^T
                gb = K.gemm(A2, g2, a_kcontig=False, b_kcontig=False)               # sum_batch a^T @ g
                return ga, gb
        elif A.ndim == 3 and B.ndim == 3 and A.shape[0] == B.shape[0]:
            y = K.gemm(A, B)

            def bw(g):
                gc = _contig(g)
                return K.gemm(gc, B, a_kcontig=True, b_kcontig=True), K.gemm(A, gc, a_kcontig=False, b_kcontig=False)
        else:
            raise NotImplementedError(f"matmul of shapes {A.shape} @ {B.shape}")
        return Tensor._make(y, (a, b), bw)

    def sum(self, axis=None, keepdims=False):
        a = self
        nd = a.data.ndim
        axes = list(range(nd)) if axis is None else [axis] if isinstance(axis, int) else list(axis)
        axes = [x % nd for x in axes] if nd else []
        out = K.reduce_sum(_contig(a.data), axes, keepdims=keepdims)

        def bw(g):
            if axis is not None and not keepdims:
                g = _contig(g).reshape(tuple(1 if d in axes else s for d, s in enumerate(a.shape)))
            return (_broadcast_to(g, a.shape),)
        return Tensor._make(out, (a,), bw)

    def mean(self, axis=None, keepdims=False):
        n = self.data.size if axis is None else self.data.shape[axis]
        return self.sum(axis, keepdims) * (1.0 / n)

    def reshape(self, *shape):
        a = self
        return Tensor._make(a.data.reshape(*shape), (a,), lambda g: (g.reshape(a.shape),))

    def transpose(self, *axes):
        a = self
        inv = tuple(np.argsort(axes))
        return Tensor._make(a.data.transpose(*axes), (a,), lambda g: (g.transpose(*inv),))

    def gelu(self):
        x = _contig(self.data)

        def bw(g):
            return (K.gelu_bwd(x, _contig(g)),)
        return Tensor._make(K.gelu_fwd(x), (self,), bw)

    def relu(self):
        x = _contig(self.data)
        return Tensor._make(K.relu_fwd(x), (self,), lambda g: (K.relu_bwd(x, _contig(g)),))

    # ------------------------------------------------------------ backward
    def backward(self, grad=None):
        """dtrain/autograd.py:151-195 over device gradients."""
        if grad is None:
            if self.data.size != 1:
                raise ValueError("backward() without a gradient needs a scalar output")
            grad = dev.full(self.data.shape, 1.0, self.data.dtype)
        elif not isinstance(grad, DeviceArray):
            grad = dev.asarray(np.asarray(grad, dtype=self.dtype))
        order, seen, users = [], set(), {}
        stack = [(self, False)]
        while stack:
            node, done = stack.pop()
            if done:
                order.append(node)
                continue
            if id(node) in seen:
                continue
            seen.add(id(node))
            stack.append((node, True))
            for p in node._parents:
                users[id(p)] = users.get(id(p), 0) + 1
                if id(p) not in seen:
                    stack.append((p, False))
        # A leaf with a grad_dest, no gradient yet and exactly one incoming
        # edge lets its producing node write the gradient straight into the
        # destination (grad_out); any other case goes through a new array.
        live = []
        for node in order:
            if node._backward is None and node.grad_dest is not None and node.requires_grad:
                if node.grad is None and users.get(id(node), 0) == 1:
                    node._dest_live = node.grad_dest
                    live.append(node)
        try:
            grads = {id(self): grad}
            for node in reversed(order):
                g = grads.pop(id(node), None)
                if g is None:
                    continue
                if node._backward is None:
                    if isinstance(g, K.SplitSum):
                        g = g.value()
                    if node.requires_grad:
                        node._dest_live = None
                        if node.grad is None:
                            node.grad = g
                        elif node.grad_dest is not None and node.grad.ptr == node.grad_dest.ptr:
                            node.grad = K.binary("add", node.grad, g, out=node.grad)  # accumulate in place
                        else:
                            node.grad = K.binary("add", node.grad, g)
                        for h in node._hooks:
                            h(node)
                    continue
                self._backprop(node, g, grads)
        finally:
            for node in live:
                node._dest_live = None
        return None

    @staticmethod
    def _backprop(node, g, grads):
        # A backward function may offer `with_addend = (i, f)`: when parent i
        # already has a pending gradient P, f(g, P) returns the parents'
        # gradients with P already added into parent i's (P + its own, the
        # order of the sum below), or None to decline.
        # a gradient left as split-K partials goes on as it is only to a
        # backward that takes it (the LayerNorm's); any other gets its value
        if isinstance(g, K.SplitSum) and not getattr(node._backward, "takes_split_sum", False):
            g = g.value()
        outs, summed = None, -1
        fuse = getattr(node._backward, "with_addend", None)
        if fuse is not None:
            i, f = fuse
            p = node._parents[i]
            if p.requires_grad and id(p) in grads:
                outs = f(g, grads[id(p)])
                summed = i if outs is not None else -1
        if outs is None:
            outs = node._backward(g)
        for j, (p, pg) in enumerate(zip(node._parents, outs)):
            if not p.requires_grad or pg is None:
                continue
            if tuple(pg.shape) != tuple(p.shape):
                raise RuntimeError(f"gradient shape {pg.shape} != {p.shape}")
            k = id(p)
            if j == summed or k not in grads:
                grads[k] = pg
            else:
                a = grads[k].value() if isinstance(grads[k], K.SplitSum) else grads[k]
                grads[k] = K.binary("add", a, pg.value() if isinstance(pg, K.SplitSum) else pg)


def grad_out(t: Tensor):
    """Where a backward function should write the gradient of `t`: its live
    grad_dest during backward() (see Tensor.grad_dest), else None."""
    return t._dest_live


# ------------------------------------------------------------ functional ops
class Indices:
    """Integer ids (token ids, positions, targets) mirrored once in HBM.

    dtrain passes index arrays as NumPy arrays (autograd.py:199, 250); every
    op accepting one also accepts an Indices, so a batch can be uploaded once
    and reused with no host-to-device copy inside a step. The embedding
    backward's stable segment order (the order np.add.at adds rows in) is
    computed on first use and kept with it.
    """

    __slots__ = ("host", "dev", "shape", "_segs", "_lo", "_hi")

    def __init__(self, idx):
        self.host = np.asarray(idx)
        if not np.issubdtype(self.host.dtype, np.integer):
            raise TypeError("indices must be integers")
        self.shape = self.host.shape
        self._lo = int(self.host.min()) if self.host.size else 0
        self._hi = int(self.host.max()) if self.host.size else -1
        self.dev = dev.from_numpy(self.host.reshape(-1).astype(np.int64))
        self._segs = None

    def check(self, n: int, what: str, allow_negative: bool):
        lo = -n if allow_negative else 0
        if self.host.size and (self._lo < lo or self._hi >= n):
            raise IndexError(f"{what} out of bounds for size {n}")

    def wrapped(self, n: int) -> "Indices":
        """Negative ids taken modulo n (NumPy indexing)."""
        if self._lo >= 0:
            return self
        return Indices(np.where(self.host < 0, self.host + n, self.host))

    def segments(self):
        """The stable sort of the indices by row, built on the device from
        the uploaded ids once (kernels.embedding_segments)."""
        if self._segs is None:
            self._segs = K.embedding_segments(self.dev)
        return self._segs


def as_indices(idx) -> Indices:
    return idx if isinstance(idx, Indices) else Indices(idx)


def embedding(weight: Tensor, idx) -> Tensor:
    """dtrain/autograd.py:199-204. `idx`: a host integer array or an Indices."""
    V = weight.shape[0]
    ix = as_indices(idx)
    ix.check(V, "index", allow_negative=True)
    ix = ix.wrapped(V)
    w = weight.data if weight.data.is_contiguous else weight.data.contiguous()
    out = K.embedding_fwd(w, ix.dev, ix.shape)

    def bw(g):
        return (K.embedding_bwd(_contig(g).reshape(-1, weight.shape[1]), V, ix.segments(), out=grad_out(weight)),)
    return Tensor._make(out, (weight,), bw)


def layer_norm(x: Tensor, w: Tensor, b: Tensor, eps=1e-5) -> Tensor:
    """dtrain/autograd.py:207-223. When the kernel that produced x already
    computed this LayerNorm of it (nn.linear(..., ln=...)), its result is used
    (the same bits)."""
    xd = _contig(x.data)
    pre, x._ln_pre = x._ln_pre, None
    if pre is not None and pre[0] is w and pre[1] is b and pre[2] == eps:
        y, mean, rstd = pre[3:]
    else:
        y, mean, rstd = K.layernorm_fwd(xd, _contig(w.data), _contig(b.data), eps)

    def bw(g, dx_addend=None):
        # g may be a kernels.SplitSum (the producer's split-K partials)
        return K.layernorm_bwd(g if isinstance(g, K.SplitSum) else _contig(g), xd, _contig(w.data), mean, rstd,
                               dw_out=grad_out(w), db_out=grad_out(b), dx_addend=dx_addend)

    def bw_add(g, pending):
        # x already has a pending gradient (the residual path): the kernel
        # writes pending + dx, the engine's own sum, in the same pass
        if isinstance(pending, K.SplitSum) or not pending.is_contiguous or pending.dtype != xd.dtype or \
                pending.shape != xd.shape:
            return None
        return bw(g, dx_addend=pending)
    bw.with_addend = (0, bw_add)
    bw.takes_split_sum = True
    t = Tensor._make(y, (x, w, b), bw)
    t._ln_out = True
    return t


def causal_attention(q: Tensor, k: Tensor, v: Tensor) -> Tensor:
    """dtrain/autograd.py:226-247 for (B, H, T, D) inputs (any strides with a
    contiguous last axis). Keeps row max/sum instead of the probabilities."""
    o, rmax, rsum = K.attn_fwd(q.data, k.data, v.data)

    def bw(g):
        gq = dev.empty(q.shape, q.dtype)
        gk = dev.empty(q.shape, q.dtype)
        gv = dev.empty(q.shape, q.dtype)
        K.attn_bwd(q.data, k.data, v.data, o, _contig(g), rmax, rsum, dq=gq, dk=gk, dv=gv)
        return gq, gk, gv
    return Tensor._make(o, (q, k, v), bw)


def cross_entropy(logits: Tensor, targets) -> Tensor:
    """dtrain/autograd.py:250-266: mean cross-entropy; `targets`: a host integer
    array or an Indices.

    With gradients enabled the logits' gradient ([rows, V], as large as the
    logits) is computed by the forward pass and held until backward runs or
    the returned loss tensor is dropped. Evaluate under `no_grad()` to skip
    it: a validation loss taken with gradients on keeps that array alive for
    as long as its loss tensor lives."""
    z = _contig(logits.data)
    V = z.shape[-1]
    t = as_indices(targets)
    t.check(V, "target", allow_negative=False)
    if not (_grad_enabled and logits.requires_grad):
        loss, rmax, rsum = K.xent_fwd(z, t.dev)
        return Tensor._make(loss, (logits,), None)
    # training: the gradient for an upstream gradient of 1 comes out of the
    # forward pass (one read of the logits); the backward rescales it in place
    # when the upstream gradient differs, and a second backward through this
    # node recomputes it from the logits and the saved row statistics
    loss, rmax, rsum, dz = K.xent_fused(z, t.dev)
    pending = [dz]

    def bw(g):
        g1 = _contig(g).reshape(1)
        if pending:
            return (K.xent_grad_scale(pending.pop(), g1),)
        return (K.xent_bwd(z, t.dev, rmax, rsum, g=g1),)
    return Tensor._make(loss, (logits,), bw)
