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
        L.sdpa_cpu_fwd.restype = i32
        L.sdpa_cpu_fwd.argtypes = [i32, vp, vp, vp, vp, vp, i32, i32, i32, i32, i32, f32, f32, i32,
                                   u64, u64, i32]
        L.sdpa_cpu_bwd.restype = i32
        L.sdpa_cpu_bwd.argtypes = [i32, vp, vp, vp, vp, vp, vp, vp, vp, vp, i32, i32, i32, i32, i32,
                                   f32, f32, i32, u64, u64, i32]
        _lib = L
    return _lib


def _code(a: np.ndarray) -> int:
    if a.dtype == np.float32:
        return 0
    if a.dtype == np.float16:
        return 1
    raise TypeError(f"float32 or float16 arrays expected, got {a.dtype}")


def _check(rc: int) -> None:
    if rc != 0:
        from . import InvalidArgumentError, status_string  # same codes and messages
        raise InvalidArgumentError(status_string(rc))


def sdpa(q, k, v, seed=0, offset=0, dropout: float = 0.0, scale: float = 1.0,
         causal_mask: bool = False, nthreads: int = 0):
    q, k, v = (np.ascontiguousarray(a) for a in (q, k, v))
    B, S_q, D_qk = q.shape
    S_kv, D_v = k.shape[1], v.shape[2]
    o = np.empty((B, S_q, D_v), dtype=q.dtype)
    stats = np.empty((B, S_q), dtype=np.float32)
    _check(library().sdpa_cpu_fwd(_code(q), q.ctypes.data, k.ctypes.data, v.ctypes.data,
                                  o.ctypes.data, stats.ctypes.data, B, S_q, S_kv, D_qk, D_v,
                                  float(scale), float(dropout), int(bool(causal_mask)),
                                  int(seed) & (2**64 - 1), int(offset) & (2**64 - 1), int(nthreads)))
    return o, stats


def sdpa_grad(q, k, v, o, stats, d_o, seed=0, offset=0, dropout: float = 0.0, scale: float = 1.0,
              causal_mask: bool = False, nthreads: int = 0):
    q, k, v, o, d_o = (np.ascontiguousarray(a) for a in (q, k, v, o, d_o))
    stats = np.ascontiguousarray(stats, dtype=np.float32)
    B, S_q, D_qk = q.shape
    S_kv, D_v = k.shape[1], v.shape[2]
    dq, dk, dv = np.empty_like(q), np.empty_like(k), np.empty_like(v)
    _check(library().sdpa_cpu_bwd(_code(q), q.ctypes.data, k.ctypes.data, v.ctypes.data,
                                  o.ctypes.data, stats.ctypes.data, d_o.ctypes.data, dq.ctypes.data,
                                  dk.ctypes.data, dv.ctypes.data, B, S_q, S_kv, D_qk, D_v,
                                  float(scale), float(dropout), int(bool(causal_mask)),
                                  int(seed) & (2**64 - 1), int(offset) & (2**64 - 1), int(nthreads)))
    return dq, dk, dv
