"""Typed wrappers: DeviceArray arguments in, libdtmi launches out.

Each function checks shapes/dtypes on the host (so a mismatched launch never
reaches the GPU), then calls the C ABI with raw device pointers. Outputs are
allocated here unless passed in.
"""
from __future__ import annotations

import ctypes as C

import numpy as np

from . import _lib
from .device import DeviceArray, empty

_c = _lib.call


def _dt(*arrays: DeviceArray) -> int:
    d = arrays[0].dtype
    for a in arrays[1:]:
        if a.dtype != d:
            raise TypeError(f"dtype mismatch: {d} vs {a.dtype}")
    return _lib.dtype_code(d)


def _contig(*arrays: DeviceArray):
    for a in arrays:
        if not a.is_contiguous:
            raise ValueError("kernel operand must be contiguous")


def _shape_arr(shape):
    return _lib.i64_array(shape)


# ------------------------------------------------------------- fills/copies
def fill(x: DeviceArray, value: float):
    if x.is_contiguous:
        _c("dtmi_fill", _lib.dtype_code(x.dtype), x.ptr, float(value), x.size)
    else:
        tmp = empty(x.shape, x.dtype)
        _c("dtmi_fill", _lib.dtype_code(x.dtype), tmp.ptr, float(value), tmp.size)
        copy_into(x, tmp)


def copy_into(dst: DeviceArray, src: DeviceArray):
    if dst.shape != src.shape:
        raise ValueError(f"copy shape mismatch {src.shape} -> {dst.shape}")
    if dst.dtype != src.dtype:
        raise TypeError("copy dtype mismatch")
    if src.size == 0:
        return
    if dst.is_contiguous and src.is_contiguous:
        _c("dtmi_memcpy_d2d", dst.ptr, src.ptr, dst.nbytes)
        return
    if dst.dtype not in (np.float32, np.float64):
        raise TypeError("strided copies support float32/float64")
    nd = dst.ndim
    _c("dtmi_copy_strided", _lib.dtype_code(dst.dtype), dst.ptr, _shape_arr(dst.strides), src.ptr,
       _shape_arr(src.strides), nd, _shape_arr(dst.shape))


# --------------------------------------------------------------- binary ops
_OPS = {"add": 0, "sub": 1, "mul": 2}


def broadcast_shape(a, b):
    return tuple(np.broadcast_shapes(tuple(a), tuple(b)))


def _bstrides(x: DeviceArray, shape):
    """Element strides of x broadcast to `shape` (0 on broadcast axes)."""
    nd = len(shape)
    pad = nd - x.ndim
    st = []
    for d in range(nd):
        if d < pad:
            st.append(0)
        else:
            s = x.shape[d - pad]
            st.append(0 if (s == 1 and shape[d] != 1) else x.strides[d - pad])
    return st


def binary(op: str, a: DeviceArray, b: DeviceArray, out: DeviceArray | None = None) -> DeviceArray:
    dt = _dt(a, b)
    shape = broadcast_shape(a.shape, b.shape)
    if out is None:
        out = empty(shape, a.dtype)
    elif out.shape != shape or not out.is_contiguous:
        raise ValueError("binary: bad output")
    if out.size == 0:
        return out
    if len(shape) == 0:
        shape_c, sa, sb = (1,), [0], [0]
    else:
        shape_c, sa, sb = shape, _bstrides(a, shape), _bstrides(b, shape)
    _c("dtmi_binary", dt, _OPS[op], out.ptr, a.ptr, _shape_arr(sa), b.ptr, _shape_arr(sb), len(shape_c),
       _shape_arr(shape_c))
    return out


def scale(x: DeviceArray, alpha: float = 1.0, alpha_dev: DeviceArray | None = None,
          out: DeviceArray | None = None) -> DeviceArray:
    _contig(x)
    if alpha_dev is not None and (alpha_dev.dtype != x.dtype or alpha_dev.size != 1):
        raise TypeError("scale: device scalar must be a 1-element array of the same dtype")
    out = out if out is not None else empty(x.shape, x.dtype)
    _c("dtmi_scale", _dt(x, out), out.ptr, x.ptr, x.size, float(alpha),
       alpha_dev.ptr if alpha_dev is not None else None)
    return out


def neg(x: DeviceArray) -> DeviceArray:
    return scale(x.contiguous(), -1.0)


# ---------------------------------------------------------- activations
def gelu_fwd(x: DeviceArray) -> DeviceArray:
    _contig(x)
    y = empty(x.shape, x.dtype)
    _c("dtmi_gelu_fwd", _dt(x), y.ptr, x.ptr, x.size)
    return y


def gelu_bwd(x: DeviceArray, dy: DeviceArray) -> DeviceArray:
    _contig(x, dy)
    if x.shape != dy.shape:
        raise ValueError("gelu_bwd shape mismatch")
    dx = empty(x.shape, x.dtype)
    _c("dtmi_gelu_bwd", _dt(x, dy), dx.ptr, x.ptr, dy.ptr, x.size)
    return dx


def relu_fwd(x: DeviceArray) -> DeviceArray:
    _contig(x)
    y = empty(x.shape, x.dtype)
    _c("dtmi_relu_fwd", _dt(x), y.ptr, x.ptr, x.size)
    return y


def relu_bwd(x: DeviceArray, dy: DeviceArray) -> DeviceArray:
    _contig(x, dy)
    dx = empty(x.shape, x.dtype)
    _c("dtmi_relu_bwd", _dt(x, dy), dx.ptr, x.ptr, dy.ptr, x.size)
    return dx


# ------------------------------------------------------------- reductions
def reduce_sum(x: DeviceArray, axes, keepdims=False) -> DeviceArray:
    axes = sorted({a % x.ndim for a in axes}) if x.ndim else []
    kept = [s for d, s in enumerate(x.shape) if d not in axes]
    out = empty(tuple(kept), x.dtype)
    if out.size == 0:
        pass
    elif x.ndim == 0:
        _c("dtmi_memcpy_d2d", out.ptr, x.ptr, x.nbytes)
    else:
        mask = (C.c_int * x.ndim)(*[1 if d in axes else 0 for d in range(x.ndim)])
        _c("dtmi_reduce_sum", _dt(x), out.ptr, x.ptr, _shape_arr(x.strides), x.ndim, _shape_arr(x.shape), mask)
    if keepdims:
        out = out.reshape(tuple(1 if d in axes else s for d, s in enumerate(x.shape)))
    return out


def colsum(x2d: DeviceArray, out: DeviceArray | None = None, accumulate=False) -> DeviceArray:
    _contig(x2d)
    rows, cols = x2d.shape
    out = out if out is not None else empty((cols,), x2d.dtype)
    _c("dtmi_colsum", _dt(x2d, out), out.ptr, x2d.ptr, rows, cols, 1 if accumulate else 0)
    return out


# ------------------------------------------------------ optimizer / buckets
def adamw(p, g, m, v, lr, b1, b2, eps, wd, b1t, b2t, gscale=1.0, gscale_dev=None):
    _contig(p, g, m, v)
    if not (p.size == g.size == m.size == v.size):
        raise ValueError("adamw: size mismatch")
    _c("dtmi_adamw", _dt(p, g, m, v), p.ptr, g.ptr, m.ptr, v.ptr, p.size, float(lr), float(b1), float(b2),
       float(eps), float(wd), float(1 - b1), float(1 - b2), float(b1t), float(b2t), float(gscale),
       gscale_dev.ptr if gscale_dev is not None else None)


def adamw_multi(ps, gs, ms, vs, lr, b1, b2, eps, wd, b1t, b2t, gscale=1.0, gscale_dev=None):
    if not ps:
        return
    dt = _dt(*ps)
    for p, g, m, v in zip(ps, gs, ms, vs):
        _contig(p, m, v)
        if g is not None:
            _contig(g)
            if g.dtype != p.dtype or g.size != p.size or m.size != p.size or v.size != p.size:
                raise ValueError("adamw_multi: size/dtype mismatch")
    n = len(ps)
    _c("dtmi_adamw_multi", dt, n, _lib.ptr_array([p.ptr for p in ps]),
       _lib.ptr_array([g.ptr if g is not None else 0 for g in gs]), _lib.ptr_array([m.ptr for m in ms]),
       _lib.ptr_array([v.ptr for v in vs]), _lib.i64_array([p.size for p in ps]), float(lr), float(b1), float(b2),
       float(eps), float(wd), float(1 - b1), float(1 - b2), float(b1t), float(b2t), float(gscale),
       gscale_dev.ptr if gscale_dev is not None else None)


def bucket_flatten(dst: DeviceArray, srcs, counts):
    """srcs: DeviceArray or None (zeros) per slot; written back to back into dst."""
    _contig(dst)
    if sum(counts) > dst.size:
        raise ValueError("bucket_flatten: sources exceed destination")
    for s, n in zip(srcs, counts):
        if s is not None:
            _contig(s)
            if s.size != n or s.dtype != dst.dtype:
                raise ValueError("bucket_flatten: source size/dtype mismatch")
    _c("dtmi_bucket_flatten", _lib.dtype_code(dst.dtype), dst.ptr,
       _lib.ptr_array([s.ptr if s is not None else 0 for s in srcs]), _lib.i64_array(counts), len(counts))


def average_blocks(n: int, dtype=np.float32) -> int:
    """Blocks (sum-of-squares partials) of a bucket average over n elements."""
    nb = C.c_int64()
    _c("dtmi_bucket_average", _lib.dtype_code(dtype), None, None, 1, int(n), int(n), 1.0, None, C.byref(nb))
    return nb.value


def bucket_average(out: DeviceArray, replicas: DeviceArray, world: int, inv_w: float,
                   partials: DeviceArray | None = None, segments=None):
    """out[i] = rank-order sum of replicas[r, i] times inv_w; replicas is a
    [W, n] array or a column slice of one (row stride >= n, unit column
    stride). The order is rank 0 first (dtrain's direct all-reduce) unless
    `segments` lists (start, first_rank) pairs: elements from `start` on are
    then summed starting at `first_rank` (dtrain's ring order)."""
    _contig(out)
    if replicas.ndim != 2 or replicas.shape[0] != world or replicas.shape[1] != out.size:
        raise ValueError("bucket_average: replicas must be [world, n]")
    if replicas.shape[1] > 1 and replicas.strides[1] != 1:
        raise ValueError("bucket_average: replica rows must be contiguous")
    stride = replicas.strides[0] if world > 1 else replicas.shape[1]
    if partials is not None and (partials.dtype != np.float64 or partials.size < average_blocks(out.size, out.dtype)):
        raise ValueError("bucket_average: partials too small")
    if segments is None:
        _c("dtmi_bucket_average", _dt(out, replicas), out.ptr, replicas.ptr, int(world), out.size, int(stride),
           float(inv_w), partials.ptr if partials is not None else None, None)
        return
    starts = _lib.i64_array([int(s) for s, _ in segments])
    firsts = (C.c_int * len(segments))(*[int(f) for _, f in segments])
    _c("dtmi_bucket_average_ring", _dt(out, replicas), out.ptr, replicas.ptr, int(world), out.size, int(stride),
       float(inv_w), starts, firsts, len(segments), partials.ptr if partials is not None else None)


def sumsq(arrays, out: DeviceArray):
    """f64 sum of squares of every array into the 1-element float64 `out`."""
    arrays = [a for a in arrays if a is not None]
    if out.dtype != np.float64 or out.size != 1:
        raise TypeError("sumsq output must be a 1-element float64 array")
    dt = _dt(*arrays) if arrays else 0
    for a in arrays:
        _contig(a)
    _c("dtmi_sumsq", dt, _lib.ptr_array([a.ptr for a in arrays]), _lib.i64_array([a.size for a in arrays]),
       len(arrays), out.ptr)


def sumsq_finish(partials: DeviceArray, count: int, out: DeviceArray, accumulate=False):
    _c("dtmi_sumsq_finish", partials.ptr, int(count), out.ptr, 1 if accumulate else 0)


def clip_scale(sumsq_dev: DeviceArray, max_norm: float, scale_out: DeviceArray, norm_out: DeviceArray | None = None):
    _c("dtmi_clip_scale", sumsq_dev.ptr, float(max_norm), scale_out.ptr,
       norm_out.ptr if norm_out is not None else None)


# -------------------------------------------------------------- layer norm
def layernorm_fwd(x: DeviceArray, w: DeviceArray, b: DeviceArray, eps: float = 1e-5):
    """Returns (y, mean, rstd); x is [..., C] (rows = product of leading dims)."""
    _contig(x, w, b)
    C_ = x.shape[-1]
    if w.shape != (C_,) or b.shape != (C_,):
        raise ValueError("layernorm: gamma/beta must be [C]")
    rows = x.size // C_ if C_ else 0
    y = empty(x.shape, x.dtype)
    mean = empty((rows,), x.dtype)
    rstd = empty((rows,), x.dtype)
    _c("dtmi_layernorm_fwd", _dt(x, w, b), y.ptr, mean.ptr, rstd.ptr, x.ptr, w.ptr, b.ptr, rows, C_, float(eps))
    return y, mean, rstd


def _out_or_new(out, shape, dtype, what):
    """A caller-provided output (contiguous, of `shape` and `dtype`) or a new array."""
    if out is None:
        return empty(shape, dtype)
    if tuple(out.shape) != tuple(shape) or out.dtype != np.dtype(dtype) or not out.is_contiguous:
        raise ValueError(f"{what}: output must be a contiguous {np.dtype(dtype).name} array of shape {tuple(shape)}")
    return out


class SplitSum:
    """A gradient left as the split-K partials of the product that made it:
    its value is ((parts[0] + parts[1]) + ...), elementwise, of shape `shape`
    (the sum pass's order). layernorm_bwd takes it as it is and adds the parts
    while it loads the rows; value() forms the array for anything else."""

    __slots__ = ("parts", "n", "shape", "dtype")

    def __init__(self, parts: DeviceArray, n: int, shape):
        self.parts, self.n, self.shape, self.dtype = parts, int(n), tuple(shape), parts.dtype

    def value(self) -> DeviceArray:
        v = self.parts[0]
        for i in range(1, self.n):
            v = binary("add", v, self.parts[i])
        return v.reshape(*self.shape)


def layernorm_bwd(dy, x: DeviceArray, w: DeviceArray, mean: DeviceArray, rstd: DeviceArray,
                  dw_out: DeviceArray | None = None, db_out: DeviceArray | None = None,
                  dx_addend: DeviceArray | None = None):
    """Returns (dx, dw, db); dw / db are written into dw_out / db_out when given.
    With dx_addend, dx = dx_addend + the input gradient (a new array). dy may
    be a SplitSum: its partials are added in the same pass."""
    if isinstance(dy, SplitSum):
        return _layernorm_bwd_parts(dy, x, w, mean, rstd, dw_out, db_out, dx_addend)
    _contig(dy, x, w, mean, rstd)
    if dy.shape != x.shape:
        raise ValueError("layernorm_bwd: dy/x shape mismatch")
    C_ = x.shape[-1]
    rows = x.size // C_
    if mean.size != rows or rstd.size != rows:
        raise ValueError("layernorm_bwd: bad row statistics")
    dx = empty(x.shape, x.dtype)
    dw = _out_or_new(dw_out, (C_,), x.dtype, "layernorm_bwd")
    db = _out_or_new(db_out, (C_,), x.dtype, "layernorm_bwd")
    if dx_addend is None:
        _c("dtmi_layernorm_bwd", _dt(dy, x, w, mean, rstd), dx.ptr, dw.ptr, db.ptr, dy.ptr, x.ptr, w.ptr, mean.ptr,
           rstd.ptr, rows, C_, 0)
    else:
        _contig(dx_addend)
        if dx_addend.shape != x.shape or dx_addend.dtype != x.dtype:
            raise ValueError("layernorm_bwd: dx_addend must match x in shape and dtype")
        _c("dtmi_layernorm_bwd_add", _dt(dy, x, w, mean, rstd, dx_addend), dx.ptr, dw.ptr, db.ptr, dy.ptr, x.ptr,
           w.ptr, mean.ptr, rstd.ptr, dx_addend.ptr, rows, C_, 0)
    return dx, dw, db


def ln_fusable_parts(dtype, cols: int) -> int:
    """How many split-K partials of dy the LayerNorm backward adds inside its
    row loads for rows of `cols` elements (16-byte aligned rows): four when a
    row is at most 4 vectors per lane, two up to 8, else none (a separate sum
    pass would run, so the product should sum its partials itself)."""
    vw = 16 // np.dtype(dtype).itemsize
    if cols % vw:
        return 0
    per_lane = -(-cols // (64 * vw))
    return 4 if per_lane <= 4 else 2 if per_lane <= 8 else 0


def _layernorm_bwd_parts(dy: SplitSum, x, w, mean, rstd, dw_out, db_out, dx_addend):
    _contig(dy.parts, x, w, mean, rstd)
    if dy.shape != x.shape or dy.dtype != x.dtype:
        raise ValueError("layernorm_bwd: dy/x shape mismatch")
    C_ = x.shape[-1]
    rows = x.size // C_
    if mean.size != rows or rstd.size != rows:
        raise ValueError("layernorm_bwd: bad row statistics")
    dx = empty(x.shape, x.dtype)
    dw = _out_or_new(dw_out, (C_,), x.dtype, "layernorm_bwd")
    db = _out_or_new(db_out, (C_,), x.dtype, "layernorm_bwd")
    if dx_addend is not None:
        _contig(dx_addend)
        if dx_addend.shape != x.shape or dx_addend.dtype != x.dtype:
            raise ValueError("layernorm_bwd: dx_addend must match x in shape and dtype")
    _c("dtmi_layernorm_bwd_parts", _dt(dy.parts, x, w, mean, rstd), dx.ptr, dw.ptr, db.ptr, dy.parts.ptr, dy.n, x.ptr,
       w.ptr, mean.ptr, rstd.ptr, dx_addend.ptr if dx_addend is not None else None, rows, C_, 0)
    return dx, dw, db


# ----------------------------------------------------------- cross entropy
def xent_fwd(logits: DeviceArray, targets: DeviceArray):
    """logits [..., V], targets int64 [...]. Returns (loss 0-d, rowmax, rowsum)."""
    _contig(logits, targets)
    V = logits.shape[-1]
    rows = logits.size // V
    if targets.dtype != np.int64 or targets.size != rows:
        raise ValueError("xent: targets must be int64 with one entry per row")
    loss = empty((), logits.dtype)
    rmax = empty((rows,), logits.dtype)
    rsum = empty((rows,), logits.dtype)
    _c("dtmi_xent_fwd", _dt(logits), loss.ptr, rmax.ptr, rsum.ptr, logits.ptr, targets.ptr, rows, V)
    return loss, rmax, rsum


def xent_bwd(logits: DeviceArray, targets: DeviceArray, rmax: DeviceArray, rsum: DeviceArray,
             g: DeviceArray | None = None, g_host: float = 1.0) -> DeviceArray:
    _contig(logits, targets, rmax, rsum)
    V = logits.shape[-1]
    rows = logits.size // V
    if g is not None and (g.size != 1 or g.dtype != logits.dtype):
        raise TypeError("xent_bwd: upstream gradient must be a 1-element array of the logits dtype")
    dz = empty(logits.shape, logits.dtype)
    _c("dtmi_xent_bwd", _dt(logits, rmax, rsum), dz.ptr, logits.ptr, rmax.ptr, rsum.ptr, targets.ptr,
       g.ptr if g is not None else None, float(g_host), rows, V)
    return dz


def xent_fused(logits: DeviceArray, targets: DeviceArray):
    """Forward plus the gradient for an upstream gradient of 1, in one pass
    over the logits where the shape allows. Returns (loss, rowmax, rowsum,
    dlogits)."""
    _contig(logits, targets)
    V = logits.shape[-1]
    rows = logits.size // V
    if targets.dtype != np.int64 or targets.size != rows:
        raise ValueError("xent: targets must be int64 with one entry per row")
    loss = empty((), logits.dtype)
    rmax = empty((rows,), logits.dtype)
    rsum = empty((rows,), logits.dtype)
    dz = empty(logits.shape, logits.dtype)
    _c("dtmi_xent_fused", _dt(logits), loss.ptr, dz.ptr, rmax.ptr, rsum.ptr, logits.ptr, targets.ptr, rows, V)
    return loss, rmax, rsum, dz


def xent_grad_scale(dz: DeviceArray, g: DeviceArray) -> DeviceArray:
    """dz *= g[0] in place unless g[0] == 1; returns dz."""
    _contig(dz, g)
    if g.size != 1 or g.dtype != dz.dtype:
        raise TypeError("xent: upstream gradient must be a 1-element array of the logits dtype")
    _c("dtmi_xent_grad_scale", _dt(dz), dz.ptr, g.ptr, dz.size)
    return dz


def softmax_bwd(p: DeviceArray, dp: DeviceArray) -> DeviceArray:
    _contig(p, dp)
    if p.shape != dp.shape:
        raise ValueError("softmax_bwd shape mismatch")
    cols = p.shape[-1]
    ds = empty(p.shape, p.dtype)
    _c("dtmi_softmax_bwd", _dt(p, dp), ds.ptr, p.ptr, dp.ptr, p.size // cols, cols)
    return ds


# --------------------------------------------------------------- embedding
def embedding_fwd(weight: DeviceArray, idx_dev: DeviceArray, out_shape) -> DeviceArray:
    _contig(weight, idx_dev)
    V, C_ = weight.shape
    out = empty(tuple(out_shape) + (C_,), weight.dtype)
    _c("dtmi_embedding_fwd", _dt(weight), out.ptr, weight.ptr, idx_dev.ptr, idx_dev.size, V, C_)
    return out


def embedding_segments(idx_dev: DeviceArray):
    """Stable sort of the device index array (int64), on the device:
    (perm, seg_start, seg_row, nseg) int32 device arrays such that segment
    s < nseg lists perm[seg_start[s] .. seg_start[s+1]), in increasing
    order, the positions holding row seg_row[s] -- np.add.at's order of
    additions. nseg (one element) stays on the device."""
    _contig(idx_dev)
    if idx_dev.dtype != np.int64:
        raise TypeError("embedding_segments: int64 indices expected")
    n = idx_dev.size
    perm, seg_row = empty((n,), np.int32), empty((n,), np.int32)
    seg_start, nseg = empty((n + 1,), np.int32), empty((1,), np.int32)
    _c("dtmi_embedding_segments", idx_dev.ptr if n else None, n, perm.ptr, seg_start.ptr, seg_row.ptr, nseg.ptr)
    return perm, seg_start, seg_row, nseg


def embedding_bwd(dout: DeviceArray, V: int, segs, out: DeviceArray | None = None) -> DeviceArray:
    """segs: the device arrays of embedding_segments; the [V, C] table
    gradient is written into `out` when given."""
    _contig(dout)
    C_ = dout.shape[-1]
    perm, seg_start, seg_row, nseg = segs
    dw = _out_or_new(out, (V, C_), dout.dtype, "embedding_bwd")
    _c("dtmi_embedding_bwd_segs", _dt(dout), dw.ptr, dout.ptr, perm.ptr, seg_start.ptr, seg_row.ptr, nseg.ptr,
       perm.size, V, C_, 1)
    return dw


# -------------------------------------------------------------------- GEMM
def gemm(A: DeviceArray, B: DeviceArray, a_kcontig=True, b_kcontig=False, bias=None, out=None, splits=0):
    """C = op(A) op(B) for 2-D or batched 3-D contiguous operands.
    A is [M, K] (a_kcontig) or [K, M]; B is [K, N] (not b_kcontig) or [N, K]."""
    _contig(A, B)
    batched = A.ndim == 3
    if batched:
        if B.ndim != 3 or B.shape[0] != A.shape[0]:
            raise ValueError("gemm: batched operands must share the batch dimension")
        nb = A.shape[0]
        a2, b2 = A.shape[1:], B.shape[1:]
    else:
        if A.ndim != 2 or B.ndim != 2:
            raise ValueError("gemm: operands must be 2-D (or 3-D batched)")
        nb = 1
        a2, b2 = A.shape, B.shape
    M, K = (a2[0], a2[1]) if a_kcontig else (a2[1], a2[0])
    K2, N = (b2[1], b2[0]) if b_kcontig else (b2[0], b2[1])
    if K != K2:
        raise ValueError(f"gemm: inner dimensions differ ({K} vs {K2})")
    shape = (nb, M, N) if batched else (M, N)
    if out is None:
        out = empty(shape, A.dtype)
    elif out.shape != shape or not out.is_contiguous:
        raise ValueError("gemm: bad output")
    if bias is not None:
        _contig(bias)
        if bias.shape != (N,):
            raise ValueError("gemm: bias must be [N]")
    lda = a2[1]
    ldb = b2[1]
    _c("dtmi_gemm", _dt(A, B, out), 1 if a_kcontig else 0, 1 if b_kcontig else 0, M, N, K, A.ptr, lda,
       a2[0] * a2[1], B.ptr, ldb, b2[0] * b2[1], out.ptr, N, M * N, nb, bias.ptr if bias is not None else None, 0,
       int(splits))
    return out


def linear_fwd(x2: DeviceArray, w: DeviceArray, b: DeviceArray | None) -> DeviceArray:
    _contig(x2, w)
    M, K = x2.shape
    K2, N = w.shape
    if K != K2:
        raise ValueError("linear: shape mismatch")
    y = empty((M, N), x2.dtype)
    _c("dtmi_linear_fwd", _dt(x2, w), y.ptr, x2.ptr, w.ptr, b.ptr if b is not None else None, M, K, N)
    return y


def linear_fwd_fused(x2: DeviceArray, w: DeviceArray, b: DeviceArray | None, residual: DeviceArray | None = None,
                     gelu: bool = False):
    """y = x @ w + b, plus `residual` (y = residual + (x @ w + b)) or, with
    gelu=True, also act = gelu(y). Returns (y, act or None)."""
    _contig(x2, w)
    M, K = x2.shape
    K2, N = w.shape
    if K != K2:
        raise ValueError("linear: shape mismatch")
    if residual is not None:
        _contig(residual)
        if residual.shape != (M, N) or residual.dtype != x2.dtype:
            raise ValueError("linear: residual must match the output")
    y = empty((M, N), x2.dtype)
    act = empty((M, N), x2.dtype) if gelu else None
    _c("dtmi_linear_fwd_fused", _dt(x2, w), y.ptr, act.ptr if act is not None else None, x2.ptr, w.ptr,
       b.ptr if b is not None else None, residual.ptr if residual is not None else None, M, K, N)
    return y, act


def linear_fwd_ln(x2: DeviceArray, w: DeviceArray, b: DeviceArray | None, residual: DeviceArray | None,
                  ln_w: DeviceArray, ln_b: DeviceArray, eps: float = 1e-5):
    """y = residual + (x @ w + b), then h = layer_norm(y; ln_w, ln_b). Returns
    (y, h, mean, rstd); the same bits as linear_fwd_fused then layernorm_fwd."""
    _contig(x2, w, ln_w, ln_b)
    M, K = x2.shape
    K2, N = w.shape
    if K != K2:
        raise ValueError("linear: shape mismatch")
    if residual is not None:
        _contig(residual)
        if residual.shape != (M, N) or residual.dtype != x2.dtype:
            raise ValueError("linear: residual must match the output")
    if ln_w.shape != (N,) or ln_b.shape != (N,):
        raise ValueError("linear_fwd_ln: LayerNorm parameters must be [N]")
    y = empty((M, N), x2.dtype)
    h = empty((M, N), x2.dtype)
    mean = empty((M,), x2.dtype)
    rstd = empty((M,), x2.dtype)
    _c("dtmi_linear_fwd_ln", _dt(x2, w, ln_w, ln_b), y.ptr, h.ptr, mean.ptr, rstd.ptr, x2.ptr, w.ptr,
       b.ptr if b is not None else None, residual.ptr if residual is not None else None, ln_w.ptr, ln_b.ptr,
       float(eps), M, K, N)
    return y, h, mean, rstd


def linear_bwd(x2: DeviceArray, w: DeviceArray, dy2: DeviceArray, need_dx=True, need_db=True,
               dw_out: DeviceArray | None = None, db_out: DeviceArray | None = None,
               gelu_pre: DeviceArray | None = None, rowdot: DeviceArray | None = None, rowdot_t: int = 1,
               dx_parts: int = 0):
    """Returns (dx, dw, db) for y = x @ w + b with x [M, K], w [K, N]; dw / db
    are written into dw_out / db_out when given. With gelu_pre (the [M, K]
    pre-activation whose GELU is x), dx is the gradient of that pre-activation.
    With rowdot (float32 [M / rowdot_t * K / 64 * rowdot_t]): also the per-64-
    column row dots of dx with x, laid out [B, K / 64, T] for rows m = b T + t
    (the attention backward's rowsum(dO * O) when x is the attention output).
    With dx_parts = n > 1, dx may come back as a SplitSum of up to n split-K
    partials instead of summed (when the product is split in 2..n)."""
    _contig(x2, w, dy2)
    M, K = x2.shape
    N = w.shape[1]
    if dy2.shape != (M, N):
        raise ValueError("linear_bwd: dy shape mismatch")
    dt = _dt(x2, w, dy2)
    dx = None
    if need_dx:
        dx = empty((M, K), x2.dtype) if dx_parts <= 1 or gelu_pre is not None or rowdot is not None else None
        if gelu_pre is not None:
            _contig(gelu_pre)
            if gelu_pre.shape != (M, K):
                raise ValueError("linear_bwd: pre-activation shape mismatch")
            _c("dtmi_linear_bwd_dx_gelu", dt, dx.ptr, dy2.ptr, w.ptr, gelu_pre.ptr, M, K, N)
        elif rowdot is not None:
            _contig(rowdot)
            if rowdot.dtype != x2.dtype or rowdot.size != M * (K // 64):
                raise ValueError("linear_bwd: rowdot must hold M * K / 64 values of x's dtype")
            _c("dtmi_linear_bwd_dx_rowdot", dt, dx.ptr, dy2.ptr, w.ptr, x2.ptr, rowdot.ptr, M, K, N, int(rowdot_t))
        elif dx_parts > 1:
            parts = empty((int(dx_parts), M, K), x2.dtype)
            n = C.c_int(1)
            _c("dtmi_linear_bwd_dx_parts", dt, parts.ptr, int(dx_parts), C.byref(n), dy2.ptr, w.ptr, M, K, N)
            dx = SplitSum(parts, n.value, (M, K)) if n.value > 1 else parts[0]
        else:
            _c("dtmi_linear_bwd_dx", dt, dx.ptr, dy2.ptr, w.ptr, M, K, N, 0)
    dw = _out_or_new(dw_out, (K, N), x2.dtype, "linear_bwd")
    db = _out_or_new(db_out, (N,), x2.dtype, "linear_bwd") if need_db else None
    _c("dtmi_linear_bwd_dw", dt, dw.ptr, db.ptr if db is not None else None, x2.ptr, dy2.ptr, M, K, N, 0)
    return dx, dw, db


# --------------------------------------------------------------- attention
def _bht_strides(x: DeviceArray):
    """(b, h, t) element strides of a (B, H, T, D) view whose last axis is contiguous."""
    if x.ndim != 4 or (x.shape[3] > 1 and x.strides[3] != 1):
        raise ValueError("attention operands must be (B, H, T, D) views with contiguous D")
    return _lib.i64_array(x.strides[:3])


def attn_fwd(q: DeviceArray, k: DeviceArray, v: DeviceArray, out: DeviceArray | None = None, scale=None):
    """Causal attention over (B, H, T, D) views. Returns (o, rowmax, rowsum);
    `out` may be a strided (B, H, T, D) view to write into."""
    if not (q.shape == k.shape == v.shape):
        raise ValueError("q, k, v shapes differ")
    B, H, T, D = q.shape
    dt = _dt(q, k, v)
    if out is None:
        out = empty(q.shape, q.dtype)
    if out.shape != q.shape:
        raise ValueError("attn_fwd: bad output")
    rowmax = empty((B, H, T), q.dtype)
    rowsum = empty((B, H, T), q.dtype)
    s = float(1.0 / np.sqrt(D)) if scale is None else float(scale)
    _c("dtmi_attn_fwd", dt, B, H, T, D, s, q.ptr, _bht_strides(q), k.ptr, _bht_strides(k), v.ptr, _bht_strides(v),
       out.ptr, _bht_strides(out), rowmax.ptr, rowsum.ptr)
    return out, rowmax, rowsum


def attn_bwd(q, k, v, o, dO, rowmax, rowsum, dq=None, dk=None, dv=None, scale=None, drow=None):
    """Returns (dq, dk, dv); each may be passed as a (B, H, T, D) view to fill.
    `drow`: rowsum(dO * O) [B, H, T] when the caller already formed it
    (linear_bwd(..., rowdot=)); the backward then skips its own row pass."""
    B, H, T, D = q.shape
    for x in (k, v, o, dO):
        if x.shape != q.shape:
            raise ValueError("attn_bwd: operand shapes differ")
    dt = _dt(q, k, v, o, dO, rowmax, rowsum)
    _contig(rowmax, rowsum)
    dq = dq if dq is not None else empty(q.shape, q.dtype)
    dk = dk if dk is not None else empty(q.shape, q.dtype)
    dv = dv if dv is not None else empty(q.shape, q.dtype)
    s = float(1.0 / np.sqrt(D)) if scale is None else float(scale)
    if drow is not None:
        _contig(drow)
        if drow.dtype != q.dtype or drow.size != B * H * T:
            raise ValueError("attn_bwd: drow must be [B, H, T] of the operands' dtype")
        _c("dtmi_attn_bwd_rowsum", dt, B, H, T, D, s, q.ptr, _bht_strides(q), k.ptr, _bht_strides(k), v.ptr,
           _bht_strides(v), o.ptr, _bht_strides(o), dO.ptr, _bht_strides(dO), rowmax.ptr, rowsum.ptr, drow.ptr,
           dq.ptr, _bht_strides(dq), dk.ptr, _bht_strides(dk), dv.ptr, _bht_strides(dv))
        return dq, dk, dv
    _c("dtmi_attn_bwd", dt, B, H, T, D, s, q.ptr, _bht_strides(q), k.ptr, _bht_strides(k), v.ptr, _bht_strides(v),
       o.ptr, _bht_strides(o), dO.ptr, _bht_strides(dO), rowmax.ptr, rowsum.ptr, dq.ptr, _bht_strides(dq), dk.ptr,
       _bht_strides(dk), dv.ptr, _bht_strides(dv))
    return dq, dk, dv


def attn_set_ds_limit(nbytes: int) -> int:
    """Bound the attention backward's dS workspace (bytes; 0 makes the dQ pass
    recompute dS). Returns the previous bound."""
    prev = C.c_int64()
    _c("dtmi_attn_set_ds_limit", int(nbytes), C.byref(prev))
    return prev.value
