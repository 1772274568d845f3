"""numpy binding of the host (CPU) kernels in ``libsdpa_cpu.so``
(``include/sdpa_cpu.h``): the op's DEVICE_CPU registration
(``sdpa/sdpa_cpu.cc:460-468``), for tensors that live in host memory.

Same interface as the GPU functions of this package, on numpy arrays:
``sdpa(q, k, v, seed, offset, dropout=, scale=, causal_mask=)`` returns
``(o, stats)`` and ``sdpa_grad(q, k, v, o, stats, d_o, seed, offset, ...)``
returns ``(dq, dk, dv)``.  Arrays are float32 or float16, C-contiguous
``[B, S, D]``.  This module is a separate device path, never a fallback of the
GPU one: it raises if its own library is missing.
"""
from __future__ import annotations

import ctypes
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libsdpa_cpu.so")
_lib = None


def library():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is missing: run __graft_entry__.build()")
        L = ctypes.CDLL(LIB_PATH)
        vp, i32, f32, u64 = ctypes.c_void_p, ctypes.c_int, ctypes.c_float, ctypes.c_uint64
        dims = ctypes.POINTER(ctypes.c_int64)
        L.sdpa_cpu_fwd.restype = i32
        L.sdpa_cpu_fwd.argtypes = [i32, vp, vp, vp, vp, vp, i32, i32, i32, i32, i32, f32, f32, i32,
                                   u64, u64, i32]
        L.sdpa_cpu_bwd.restype = i32
        L.sdpa_cpu_bwd.argtypes = [i32, vp, vp, vp, vp, vp, vp, vp, vp, vp, i32, i32, i32, i32, i32,
                                   f32, f32, i32, u64, u64, i32]
        L.sdpa_cpu_status_string.restype = ctypes.c_char_p
        L.sdpa_cpu_status_string.argtypes = [i32]
        L.sdpa_cpu_check_fwd.restype = i32
        L.sdpa_cpu_check_fwd.argtypes = [i32, dims, i32, dims, i32, dims, i32, i32, i32]
        L.sdpa_cpu_check_bwd.restype = i32
        L.sdpa_cpu_check_bwd.argtypes = [i32, dims] * 6 + [i32, i32, i32]
        _lib = L
    return _lib


def _error(msg: str):
    from . import InvalidArgumentError  # the error class of the op (no GPU library needed)
    return InvalidArgumentError(msg)


def _check(rc: int) -> None:
    if rc != 0:
        raise _error(library().sdpa_cpu_status_string(rc).decode())


def _dims(a) -> tuple:
    shape = tuple(int(d) for d in np.shape(a))
    return len(shape), (ctypes.c_int64 * max(1, len(shape)))(*shape)


def _code(arrays, names) -> int:
    """dtype code of the op's T: every array float32, or every one float16."""
    dt = arrays[0].dtype
    if dt not in (np.float32, np.float16):
        raise _error(f"T must be half or float, got {dt}")
    for a, n in zip(arrays, names):
        if a.dtype != dt:
            raise _error(f"{n} has dtype {a.dtype}, expected {dt} (all of {', '.join(names)} share T)")
    return 0 if dt == np.float32 else 1


def _u64(x) -> int:
    return int(np.asarray(x).item()) & (2**64 - 1)


def sdpa(q, k, v, seed=0, offset=0, dropout: float = 0.0, scale: float = 1.0,
         causal_mask: bool = False, nthreads: int = 0):
    """Forward op ``Sdpa`` on host arrays: returns ``(o, stats)``.  Arguments
    are checked as the op checks them (ranks, batch / sequence / feature
    sizes, scalar seed and offset; sdpa/sdpa_cpu.cc:37-69) before any data is
    read."""
    q, k, v = (np.ascontiguousarray(a) for a in (q, k, v))
    code = _code((q, k, v), ("q", "k", "v"))
    L = library()
    _check(L.sdpa_cpu_check_fwd(*_dims(q), *_dims(k), *_dims(v), np.ndim(seed), np.ndim(offset),
                                int(bool(causal_mask))))
    B, S_q, D_qk = q.shape
    S_kv, D_v = k.shape[1], v.shape[2]
    o = np.empty((B, S_q, D_v), dtype=q.dtype)
    stats = np.empty((B, S_q), dtype=np.float32)
    _check(L.sdpa_cpu_fwd(code, q.ctypes.data, k.ctypes.data, v.ctypes.data, o.ctypes.data,
                          stats.ctypes.data, B, S_q, S_kv, D_qk, D_v, float(scale), float(dropout),
                          int(bool(causal_mask)), _u64(seed), _u64(offset), int(nthreads)))
    return o, stats


def sdpa_grad(q, k, v, o, stats, d_o, seed=0, offset=0, dropout: float = 0.0, scale: float = 1.0,
              causal_mask: bool = False, nthreads: int = 0):
    """Gradient op ``SdpaGrad`` on host arrays: returns ``(dq, dk, dv)``.
    Checked as the op checks them (sdpa/sdpa_cpu.cc:116-168); stats must be
    float32, as the op's ``stats: float`` input."""
    q, k, v, o, d_o, stats = (np.ascontiguousarray(a) for a in (q, k, v, o, d_o, stats))
    code = _code((q, k, v, o, d_o), ("q", "k", "v", "o", "d_o"))
    if stats.dtype != np.float32:
        raise _error(f"stats must be float32, got {stats.dtype}")
    L = library()
    _check(L.sdpa_cpu_check_bwd(*_dims(q), *_dims(k), *_dims(v), *_dims(o), *_dims(stats), *_dims(d_o),
                                np.ndim(seed), np.ndim(offset), int(bool(causal_mask))))
    B, S_q, D_qk = q.shape
    S_kv, D_v = k.shape[1], v.shape[2]
    dq, dk, dv = np.empty_like(q), np.empty_like(k), np.empty_like(v)
    _check(L.sdpa_cpu_bwd(code, q.ctypes.data, k.ctypes.data, v.ctypes.data, o.ctypes.data,
                          stats.ctypes.data, d_o.ctypes.data, dq.ctypes.data, dk.ctypes.data,
                          dv.ctypes.data, B, S_q, S_kv, D_qk, D_v, float(scale), float(dropout),
                          int(bool(causal_mask)), _u64(seed), _u64(offset), int(nthreads)))
    return dq, dk, dv
