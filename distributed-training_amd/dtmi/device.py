"""Device arrays: the HBM buffers behind every dtmi Tensor.

dtrain's Tensor holds a NumPy ndarray in `.data` (dtrain/autograd.py:43). Here
`.data` is a DeviceArray: a view (shape, element strides, byte offset, dtype)
onto a block of device memory that libdtmi allocated and owns. Python holds the
block through a reference-counted handle that returns it to the library's pool
when the last view goes away.

Views are free: reshape of a contiguous array, transpose/swapaxes, slicing along
the first axis and flat slicing are metadata only. Kernels read contiguous
arrays; `.contiguous()` materialises a strided view with one copy kernel.
`np.asarray(device_array)` and `.numpy()` copy to the host.
"""
from __future__ import annotations

import ctypes as C
from math import prod

import numpy as np

from . import _lib

_ITEMSIZE = {np.dtype(np.float32): 4, np.dtype(np.float64): 8, np.dtype(np.int64): 8, np.dtype(np.int32): 4}


class Block:
    """One libdtmi allocation. Freed (returned to the pool) on garbage collection."""

    __slots__ = ("ptr", "nbytes", "__weakref__")

    def __init__(self, nbytes: int):
        p = C.c_void_p()
        _lib.call("dtmi_malloc", C.byref(p), max(int(nbytes), 1))
        self.ptr = p.value
        self.nbytes = int(nbytes)

    def __del__(self):
        L = _lib._lib
        if L is not None and self.ptr:
            L.dtmi_free(self.ptr)
            self.ptr = None


def _contig_strides(shape):
    st, acc = [], 1
    for s in reversed(shape):
        st.append(acc)
        acc *= int(s)
    return tuple(reversed(st))


class DeviceArray:
    __slots__ = ("block", "offset", "shape", "strides", "dtype", "__weakref__")
    __array_priority__ = 100

    def __init__(self, block: Block, shape, dtype, offset: int = 0, strides=None):
        self.block = block
        self.shape = tuple(int(s) for s in shape)
        self.dtype = np.dtype(dtype)
        self.offset = int(offset)  # bytes
        self.strides = tuple(strides) if strides is not None else _contig_strides(self.shape)  # elements

    # ------------------------------------------------------------ metadata
    @property
    def itemsize(self) -> int:
        return _ITEMSIZE[self.dtype]

    @property
    def size(self) -> int:
        return prod(self.shape)

    @property
    def ndim(self) -> int:
        return len(self.shape)

    @property
    def nbytes(self) -> int:
        return self.size * self.itemsize

    @property
    def ptr(self) -> int:
        return self.block.ptr + self.offset

    @property
    def is_contiguous(self) -> bool:
        exp = 1
        for s, st in zip(reversed(self.shape), reversed(self.strides)):
            if s != 1 and st != exp:
                return False
            exp *= s
        return True

    def __len__(self):
        if not self.shape:
            raise TypeError("len() of a 0-d array")
        return self.shape[0]

    def __repr__(self):
        return f"DeviceArray(shape={self.shape}, dtype={self.dtype}, contiguous={self.is_contiguous})"

    # ------------------------------------------------------------- host io
    def numpy(self) -> np.ndarray:
        src = self if self.is_contiguous else self.contiguous()
        out = np.empty(self.shape, self.dtype)
        if out.nbytes:
            _lib.call("dtmi_memcpy_d2h", out.ctypes.data, src.ptr, out.nbytes)
        return out

    def __array__(self, dtype=None, copy=None):
        a = self.numpy()
        return a if dtype is None else a.astype(dtype, copy=False)

    def item(self):
        return self.numpy().item()

    def __float__(self):
        return float(self.numpy())

    # --------------------------------------------------------------- views
    def reshape(self, *shape) -> "DeviceArray":
        if len(shape) == 1 and isinstance(shape[0], (tuple, list)):
            shape = tuple(shape[0])
        shape = list(int(s) for s in shape)
        if shape.count(-1) > 1:
            raise ValueError("can only specify one unknown dimension")
        if -1 in shape:
            known = prod(s for s in shape if s != -1)
            shape[shape.index(-1)] = self.size // known if known else 0
        if prod(shape) != self.size:
            raise ValueError(f"cannot reshape array of size {self.size} into shape {tuple(shape)}")
        src = self if self.is_contiguous else self.contiguous()
        return DeviceArray(src.block, shape, src.dtype, src.offset)

    def transpose(self, *axes) -> "DeviceArray":
        if len(axes) == 1 and isinstance(axes[0], (tuple, list)):
            axes = tuple(axes[0])
        if not axes:
            axes = tuple(reversed(range(self.ndim)))
        axes = tuple(a % self.ndim for a in axes)
        if sorted(axes) != list(range(self.ndim)):
            raise ValueError(f"axes {axes} do not permute {self.ndim} dimensions")
        return DeviceArray(self.block, [self.shape[a] for a in axes], self.dtype, self.offset,
                           [self.strides[a] for a in axes])

    def swapaxes(self, a: int, b: int) -> "DeviceArray":
        ax = list(range(self.ndim))
        ax[a], ax[b] = ax[b], ax[a]
        return self.transpose(ax)

    @property
    def T(self) -> "DeviceArray":
        return self.transpose()

    def __getitem__(self, idx) -> "DeviceArray":
        """Integer or unit-step slice along the first axis (a view)."""
        if not isinstance(idx, tuple):
            idx = (idx,)
        if len(idx) != 1:
            raise IndexError("DeviceArray supports indexing along the first axis only")
        i = idx[0]
        n0 = self.shape[0]
        if isinstance(i, (int, np.integer)):
            i = int(i)
            if i < 0:
                i += n0
            if not 0 <= i < n0:
                raise IndexError(f"index {idx[0]} out of range for axis of size {n0}")
            return DeviceArray(self.block, self.shape[1:], self.dtype, self.offset + i * self.strides[0] * self.itemsize,
                               self.strides[1:])
        if isinstance(i, slice):
            lo, hi, step = i.indices(n0)
            if step != 1:
                raise IndexError("DeviceArray slices must have step 1")
            hi = max(hi, lo)
            return DeviceArray(self.block, (hi - lo,) + self.shape[1:], self.dtype,
                               self.offset + lo * self.strides[0] * self.itemsize, self.strides)
        raise IndexError(f"unsupported index {i!r}")

    def __setitem__(self, idx, value):
        view = self[idx]
        view.assign(value)

    # -------------------------------------------------------------- copies
    def assign(self, value) -> "DeviceArray":
        """Copy `value` (DeviceArray, ndarray or scalar) into this view in place."""
        from . import kernels as K
        if isinstance(value, DeviceArray):
            if value.shape != self.shape:
                raise ValueError(f"shape mismatch {value.shape} -> {self.shape}")
            K.copy_into(self, value)
        elif np.isscalar(value):
            K.fill(self, float(value))
        else:
            a = np.ascontiguousarray(np.broadcast_to(np.asarray(value, dtype=self.dtype), self.shape))
            if not self.is_contiguous:
                tmp = from_numpy(a)
                K.copy_into(self, tmp)
            elif a.nbytes:
                _lib.call("dtmi_memcpy_h2d", self.ptr, a.ctypes.data, a.nbytes)
        return self

    def copy(self) -> "DeviceArray":
        from . import kernels as K
        out = empty(self.shape, self.dtype)
        K.copy_into(out, self)
        return out

    def contiguous(self) -> "DeviceArray":
        return self if self.is_contiguous else self.copy()

    def fill_(self, value: float) -> "DeviceArray":
        from . import kernels as K
        K.fill(self, float(value))
        return self

    def zero_(self) -> "DeviceArray":
        return self.fill_(0.0)


# ----------------------------------------------------------------- factories
def empty(shape, dtype=np.float32) -> DeviceArray:
    if isinstance(shape, (int, np.integer)):
        shape = (int(shape),)
    dt = np.dtype(dtype)
    n = prod(shape)
    return DeviceArray(Block(n * _ITEMSIZE[dt]), shape, dt)


def zeros(shape, dtype=np.float32) -> DeviceArray:
    return empty(shape, dtype).zero_()


def full(shape, value, dtype=np.float32) -> DeviceArray:
    return empty(shape, dtype).fill_(value)


def from_numpy(a) -> DeviceArray:
    a = np.ascontiguousarray(a)
    if a.dtype not in _ITEMSIZE:
        raise TypeError(f"unsupported dtype {a.dtype}")
    out = empty(a.shape, a.dtype)
    if a.nbytes:
        _lib.call("dtmi_memcpy_h2d", out.ptr, a.ctypes.data, a.nbytes)
    return out


def asarray(x, dtype=None) -> DeviceArray:
    if isinstance(x, DeviceArray):
        if dtype is not None and np.dtype(dtype) != x.dtype:
            raise TypeError("DeviceArray dtype conversion is not supported")
        return x
    a = np.asarray(x, dtype=dtype)
    return from_numpy(a)
