"""ctypes binding of libdtmi.so (the C ABI declared in include/dtmi.h).

There is no fallback: if the library or a GPU is missing, `lib()` raises. The
library is loaded lazily, so importing the package (and the host-only logic in
it, such as bucket layouts) works on a machine without a GPU.
"""
from __future__ import annotations

import ctypes as C
import os
import re
from pathlib import Path

import numpy as np

LIB_PATH = Path(__file__).resolve().parent / "libdtmi.so"
HEADER = Path(__file__).resolve().parents[2] / "include" / "dtmi.h"

F32, F64 = 0, 1
FAM = {"gemm": 0, "attn_fwd": 1, "attn_bwd": 2, "adamw": 3, "bucket_avg": 4, "ln_bwd": 5, "gelu_bwd": 6,
       "xent": 7, "sumsq": 8, "flatten": 9, "other": 10}

vp, i32, i64, f64, sz = C.c_void_p, C.c_int, C.c_int64, C.c_double, C.c_size_t
pvp, pi64, pf64, psz = C.POINTER(C.c_void_p), C.POINTER(C.c_int64), C.POINTER(C.c_double), C.POINTER(C.c_size_t)

# name -> argtypes (restype is always int status, except dtmi_last_error)
SIGNATURES: dict[str, list] = {
    "dtmi_init": [i32],
    "dtmi_device_info": [C.POINTER(C.c_int), psz, C.c_char_p, i32],
    "dtmi_malloc": [pvp, sz],
    "dtmi_free": [vp],
    "dtmi_empty_cache": [],
    "dtmi_memory_stats": [psz, psz, psz],
    "dtmi_memcpy_h2d": [vp, vp, sz],
    "dtmi_memcpy_d2h": [vp, vp, sz],
    "dtmi_memcpy_d2d": [vp, vp, sz],
    "dtmi_fill": [i32, vp, f64, i64],
    "dtmi_zero_bytes": [vp, sz],
    "dtmi_sync": [],
    "dtmi_event_create": [pvp],
    "dtmi_event_record": [vp],
    "dtmi_event_elapsed_ms": [vp, vp, C.POINTER(C.c_float)],
    "dtmi_event_destroy": [vp],
    "dtmi_timing_enable": [i32],
    "dtmi_timing_read": [i32, pi64, pf64, pf64],
    "dtmi_adamw": [i32, vp, vp, vp, vp, i64, f64, f64, f64, f64, f64, f64, f64, f64, f64, f64, vp],
    "dtmi_adamw_multi": [i32, i32, pvp, pvp, pvp, pvp, pi64, f64, f64, f64, f64, f64, f64, f64, f64, f64, f64, vp],
    "dtmi_bucket_flatten": [i32, vp, pvp, pi64, i32],
    "dtmi_bucket_average": [i32, vp, vp, i32, i64, i64, f64, vp, pi64],
    "dtmi_bucket_average_ring": [i32, vp, vp, i32, i64, i64, f64, pi64, C.POINTER(C.c_int), i32, vp],
    "dtmi_sumsq": [i32, pvp, pi64, i32, vp],
    "dtmi_sumsq_finish": [vp, i64, vp, i32],
    "dtmi_clip_scale": [vp, f64, vp, vp],
    "dtmi_copy_strided": [i32, vp, pi64, vp, pi64, i32, pi64],
    "dtmi_binary": [i32, i32, vp, vp, pi64, vp, pi64, i32, pi64],
    "dtmi_scale": [i32, vp, vp, i64, f64, vp],
    "dtmi_gelu_fwd": [i32, vp, vp, i64],
    "dtmi_gelu_bwd": [i32, vp, vp, vp, i64],
    "dtmi_relu_fwd": [i32, vp, vp, i64],
    "dtmi_relu_bwd": [i32, vp, vp, vp, i64],
    "dtmi_reduce_sum": [i32, vp, vp, pi64, i32, pi64, C.POINTER(C.c_int)],
    "dtmi_colsum": [i32, vp, vp, i64, i64, i32],
    "dtmi_layernorm_fwd": [i32, vp, vp, vp, vp, vp, vp, i64, i64, f64],
    "dtmi_layernorm_bwd": [i32, vp, vp, vp, vp, vp, vp, vp, vp, i64, i64, i32],
    "dtmi_layernorm_bwd_add": [i32, vp, vp, vp, vp, vp, vp, vp, vp, vp, i64, i64, i32],
    "dtmi_layernorm_bwd_parts": [i32, vp, vp, vp, vp, i32, vp, vp, vp, vp, vp, i64, i64, i32],
    "dtmi_linear_bwd_dx_parts": [i32, vp, i32, C.POINTER(C.c_int), vp, vp, i64, i64, i64],
    "dtmi_layernorm_bwd_noalloc": [i32, vp, vp, vp, vp, vp, vp, vp, vp, i64, i64, i32],
    "dtmi_xent_fwd": [i32, vp, vp, vp, vp, vp, i64, i64],
    "dtmi_xent_bwd": [i32, vp, vp, vp, vp, vp, vp, f64, i64, i64],
    "dtmi_xent_fused": [i32, vp, vp, vp, vp, vp, vp, i64, i64],
    "dtmi_xent_grad_scale": [i32, vp, vp, i64],
    "dtmi_softmax_bwd": [i32, vp, vp, vp, i64, i64],
    "dtmi_embedding_fwd": [i32, vp, vp, vp, i64, i64, i64],
    "dtmi_embedding_bwd": [i32, vp, vp, vp, vp, vp, i32, i64, i64, i32],
    "dtmi_embedding_segments": [vp, i64, vp, vp, vp, vp],
    "dtmi_embedding_bwd_segs": [i32, vp, vp, vp, vp, vp, vp, i64, i64, i64, i32],
    "dtmi_gemm": [i32, i32, i32, i64, i64, i64, vp, i64, i64, vp, i64, i64, vp, i64, i64, i64, vp, i32, i32],
    "dtmi_set_gemm_math": [i32],
    "dtmi_get_gemm_math": [vp],
    "dtmi_linear_fwd": [i32, vp, vp, vp, vp, i64, i64, i64],
    "dtmi_linear_bwd_dx": [i32, vp, vp, vp, i64, i64, i64, i32],
    "dtmi_linear_bwd_dw": [i32, vp, vp, vp, vp, i64, i64, i64, i32],
    "dtmi_linear_fwd_fused": [i32, vp, vp, vp, vp, vp, vp, i64, i64, i64],
    "dtmi_linear_fwd_ln": [i32, vp, vp, vp, vp, vp, vp, vp, vp, vp, vp, f64, i64, i64, i64],
    "dtmi_linear_bwd_dx_gelu": [i32, vp, vp, vp, vp, i64, i64, i64],
    "dtmi_linear_bwd_dx_rowdot": [i32, vp, vp, vp, vp, vp, i64, i64, i64, i64],
    "dtmi_attn_fwd": [i32, i64, i64, i64, i64, f64, vp, pi64, vp, pi64, vp, pi64, vp, pi64, vp, vp],
    "dtmi_attn_bwd": [i32, i64, i64, i64, i64, f64, vp, pi64, vp, pi64, vp, pi64, vp, pi64, vp, pi64, vp, vp,
                      vp, pi64, vp, pi64, vp, pi64],
    "dtmi_attn_bwd_rowsum": [i32, i64, i64, i64, i64, f64, vp, pi64, vp, pi64, vp, pi64, vp, pi64, vp, pi64, vp, vp,
                             vp, vp, pi64, vp, pi64, vp, pi64],
    "dtmi_attn_set_ds_limit": [i64, pi64],
}

_lib = None
_initialised = False


class DtmiError(RuntimeError):
    """A libdtmi call returned a non-zero status."""


def header_symbols() -> list[str]:
    """Function names declared in include/dtmi.h (used by the ABI tests)."""
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(dtmi_\w+)\s*\(", text)))


def load(path: Path | str | None = None):
    """Load the shared library and attach prototypes (no device work)."""
    global _lib
    if _lib is not None:
        return _lib
    p = Path(path) if path else LIB_PATH
    if not p.exists():
        raise ImportError(f"libdtmi.so not found at {p}; build it with `python distributed-training_amd/build.py` "
                          "or __graft_entry__.build()")
    lib = C.CDLL(str(p), mode=C.RTLD_GLOBAL)
    lib.dtmi_last_error.restype = C.c_char_p
    lib.dtmi_last_error.argtypes = []
    for name, args in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = C.c_int
        fn.argtypes = args
    _lib = lib
    return lib


def lib():
    """The library, initialised on device DTMI_DEVICE (default 0), with the
    float32 GEMM arithmetic DTMI_GEMM_MATH ("f32", the default, or "bf16x6")."""
    global _initialised
    L = load()
    if not _initialised:
        rc = L.dtmi_init(int(os.environ.get("DTMI_DEVICE", "0")))
        if rc != 0:
            raise DtmiError(f"dtmi_init failed ({rc}): {L.dtmi_last_error().decode()}")
        mode = os.environ.get("DTMI_GEMM_MATH", "f32")
        if mode not in GEMM_MATH:
            raise ValueError(f"DTMI_GEMM_MATH={mode!r}; expected one of {sorted(GEMM_MATH)}")
        rc = L.dtmi_set_gemm_math(GEMM_MATH[mode])
        if rc != 0:
            raise DtmiError(f"dtmi_set_gemm_math failed ({rc}): {L.dtmi_last_error().decode()}")
        _initialised = True
    return L


def call(name: str, *args):
    rc = getattr(lib(), name)(*args)
    if rc != 0:
        raise DtmiError(f"{name} failed ({rc}): {_lib.dtmi_last_error().decode()}")


def dtype_code(dt) -> int:
    dt = np.dtype(dt)
    if dt == np.float32:
        return F32
    if dt == np.float64:
        return F64
    raise TypeError(f"libdtmi computes in float32 or float64, not {dt}")


def ptr_array(ptrs) -> C.Array:
    return (C.c_void_p * max(1, len(ptrs)))(*[C.c_void_p(p) if p else None for p in ptrs])


def i64_array(vals) -> C.Array:
    return (C.c_int64 * max(1, len(vals)))(*[int(v) for v in vals])


def sync():
    call("dtmi_sync")


def timing_enable(on: bool):
    call("dtmi_timing_enable", 1 if on else 0)


def timing_read(family: str):
    n, ms, work = C.c_int64(), C.c_double(), C.c_double()
    call("dtmi_timing_read", FAM[family], C.byref(n), C.byref(ms), C.byref(work))
    return n.value, ms.value, work.value


GEMM_MATH = {"f32": 0, "bf16x6": 1}


def set_gemm_math(mode: str):
    """Arithmetic of the float32 GEMMs: "f32" (float32 MFMA, the default) or
    "bf16x6" (each operand split exactly into three bf16 parts, the six
    largest partial products on the bf16 MFMA, float32 accumulation)."""
    if mode not in GEMM_MATH:
        raise ValueError(f"unknown GEMM math {mode!r}; expected one of {sorted(GEMM_MATH)}")
    call("dtmi_set_gemm_math", GEMM_MATH[mode])


def gemm_math() -> str:
    m = C.c_int()
    call("dtmi_get_gemm_math", C.byref(m))
    return {v: k for k, v in GEMM_MATH.items()}[m.value]


class use_gemm_math:
    """with use_gemm_math("bf16x6"): ... -- the previous mode is restored on exit."""

    def __init__(self, mode: str):
        self.mode = mode

    def __enter__(self):
        self.prev = gemm_math()
        set_gemm_math(self.mode)
        return self

    def __exit__(self, *exc):
        set_gemm_math(self.prev)
        return False


def memory_stats():
    a, b, c = C.c_size_t(), C.c_size_t(), C.c_size_t()
    call("dtmi_memory_stats", C.byref(a), C.byref(b), C.byref(c))
    return {"in_use": a.value, "cached": b.value, "peak": c.value}


def device_info():
    cus, mem = C.c_int(), C.c_size_t()
    name = C.create_string_buffer(256)
    call("dtmi_device_info", C.byref(cus), C.byref(mem), name, 256)
    return {"num_cus": cus.value, "hbm_bytes": mem.value, "name": name.value.decode()}
