"""oracle.py -- TEST INFRASTRUCTURE ONLY.

numpy front end for the CPU restatement of the reference CPU path
(``sdpa_oracle.cc``; reference ``sdpa/sdpa_cpu.cc:197-457``).  Only tests/,
``__graft_entry__.smoke()`` and ``bench.py``'s cpu_baseline leg import this
module; the product path never does.

Arrays are numpy, C-contiguous, ``[B, S, D]`` row-major like the reference's
tensors.  fp16 arrays are passed as ``numpy.float16`` (bit-identical to the
reference's Eigen::half storage).
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "libsdpa_oracle.so")
_lib = None

_u64 = ctypes.c_uint64
_i64 = ctypes.c_int64
_int = ctypes.c_int
_flt = ctypes.c_float
_vp = ctypes.c_void_p


def build() -> None:
    """Compile the oracle with its Makefile (g++ -O2, as reference build.sh:46)."""
    subprocess.run(["make", "-s", "-B", "-C", _HERE, "libsdpa_oracle.so"], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = ctypes.CDLL(_LIB_PATH)
        L.oracle_rng_bits.restype = ctypes.c_uint32
        L.oracle_rng_bits.argtypes = [_u64, _u64, _i64, _int, _int, _int, _int]
        L.oracle_rng_uniform.restype = _flt
        L.oracle_rng_uniform.argtypes = [_u64, _u64, _i64, _int, _int, _int, _int]
        L.oracle_keep_mask.restype = None
        L.oracle_keep_mask.argtypes = [_int, _int, _int, _flt, _u64, _u64, _vp, _int]
        L.oracle_float_to_half.restype = ctypes.c_uint16
        L.oracle_float_to_half.argtypes = [_flt]
        L.oracle_half_to_float.restype = _flt
        L.oracle_half_to_float.argtypes = [ctypes.c_uint16]
        L.oracle_float_to_half_n.restype = None
        L.oracle_float_to_half_n.argtypes = [_vp, _vp, ctypes.c_size_t]
        L.oracle_half_to_float_n.restype = None
        L.oracle_half_to_float_n.argtypes = [_vp, _vp, ctypes.c_size_t]
        L.oracle_sdpa_fwd.restype = _int
        L.oracle_sdpa_fwd.argtypes = [_int, _vp, _vp, _vp, _vp, _vp, _int, _int, _int, _int, _int,
                                      _int, _flt, _flt, _u64, _u64, _int, _int, _int, _int, _int]
        L.oracle_sdpa_bwd.restype = _int
        L.oracle_sdpa_bwd.argtypes = [_int, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _int,
                                      _int, _int, _int, _int, _int, _flt, _flt, _u64, _u64, _int,
                                      _int, _int, _int, _int, _int, _int, _int, _int]
        _lib = L
    return _lib


def default_threads() -> int:
    return max(1, min(os.cpu_count() or 1, 16))


def rng_bits(seed: int, offset: int, b: int, i: int, j: int, S_q: int, S_kv: int) -> int:
    return int(lib().oracle_rng_bits(seed, offset, b, i, j, S_q, S_kv))


def rng_uniform(seed: int, offset: int, b: int, i: int, j: int, S_q: int, S_kv: int) -> float:
    return float(lib().oracle_rng_uniform(seed, offset, b, i, j, S_q, S_kv))


def keep_mask(B: int, S_q: int, S_kv: int, dropout: float, seed: int, offset: int,
              nthreads: int | None = None) -> np.ndarray:
    """uint8 [B, S_q, S_kv]: 1 where the reference keeps the element."""
    out = np.empty((B, S_q, S_kv), dtype=np.uint8)
    lib().oracle_keep_mask(B, S_q, S_kv, dropout, seed, offset, out.ctypes.data,
                           nthreads or default_threads())
    return out


def float_to_half_bits(x: np.ndarray) -> np.ndarray:
    """uint16 bit patterns of the oracle's float -> half conversion (RNE)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, dtype=np.uint16)
    lib().oracle_float_to_half_n(x.ctypes.data, out.ctypes.data, x.size)
    return out


def half_bits_to_float(h: np.ndarray) -> np.ndarray:
    """float32 values of the oracle's half -> float conversion."""
    h = np.ascontiguousarray(h, dtype=np.uint16)
    out = np.empty(h.shape, dtype=np.float32)
    lib().oracle_half_to_float_n(h.ctypes.data, out.ctypes.data, h.size)
    return out


def _dtype_code(a: np.ndarray) -> int:
    if a.dtype == np.float32:
        return 0
    if a.dtype == np.float16:
        return 1
    raise TypeError(f"oracle supports float32/float16, got {a.dtype}")


def _c(a: np.ndarray) -> np.ndarray:
    return np.ascontiguousarray(a)


def _span(sp):
    """(begin, end[, step]) -> three ints; None -> everything."""
    if sp is None:
        return (0, -1, 1)
    sp = tuple(int(x) for x in sp)
    return sp + (1,) if len(sp) == 2 else sp


def sdpa_fwd(q, k, v, *, scale=1.0, dropout=0.0, causal_mask=False, seed=0, offset=0,
             gpu_gates=True, nthreads=None, rows=None):
    """Reference forward (sdpa_cpu.cc:213-320). Returns (o [B,S_q,D_v] in q.dtype, stats f32 [B,S_q]).

    rows=(i0, i1[, step]) computes only query rows i0, i0 + step, ... < i1
    (a timing sample, or a cheap check of every batch); other rows of the
    outputs are left uninitialised."""
    q, k, v = _c(q), _c(k), _c(v)
    assert q.dtype == k.dtype == v.dtype
    B, S_q, D_qk = q.shape
    S_kv, D_v = k.shape[1], v.shape[2]
    o = np.empty((B, S_q, D_v), dtype=q.dtype)
    stats = np.empty((B, S_q), dtype=np.float32)
    rc = lib().oracle_sdpa_fwd(_dtype_code(q), q.ctypes.data, k.ctypes.data, v.ctypes.data,
                               o.ctypes.data, stats.ctypes.data, B, S_q, S_kv, D_qk, D_v,
                               int(bool(causal_mask)), float(dropout), float(scale), int(seed),
                               int(offset), int(bool(gpu_gates)), nthreads or default_threads(),
                               *_span(rows))
    assert rc == 0
    return o, stats


def sdpa_bwd(q, k, v, o, stats, d_o, *, scale=1.0, dropout=0.0, causal_mask=False, seed=0,
             offset=0, gpu_gates=True, accumulate_kv_in_t=False, nthreads=None, rows=None,
             keys=None):
    """Reference backward (sdpa_cpu.cc:322-457). Returns (dq, dk, dv) in q.dtype.

    rows / keys = (begin, end[, step]) restrict the (query, key) pairs that
    are visited: dq of a row is complete only with every key visited, dk / dv
    of a key only with every row visited."""
    q, k, v, o, d_o = _c(q), _c(k), _c(v), _c(o), _c(d_o)
    stats = np.ascontiguousarray(stats, dtype=np.float32)
    B, S_q, D_qk = q.shape
    S_kv, D_v = k.shape[1], v.shape[2]
    dq = np.empty_like(q)
    dk = np.empty_like(k)
    dv = np.empty_like(v)
    rc = lib().oracle_sdpa_bwd(_dtype_code(q), q.ctypes.data, k.ctypes.data, v.ctypes.data,
                               o.ctypes.data, stats.ctypes.data, d_o.ctypes.data, dq.ctypes.data,
                               dk.ctypes.data, dv.ctypes.data, B, S_q, S_kv, D_qk, D_v,
                               int(bool(causal_mask)), float(dropout), float(scale), int(seed),
                               int(offset), int(bool(gpu_gates)), int(bool(accumulate_kv_in_t)),
                               nthreads or default_threads(), *_span(rows), *_span(keys))
    assert rc == 0
    return dq, dk, dv


def sdpa_fwd_gate(q, k, v, **kw):
    """Gating oracle: the fp32 instantiation fed the (possibly fp16-exact) inputs.

    For fp16 inputs the values are widened exactly to fp32 and o is rounded
    back to fp16 at the end, like the output cast of sdpa_cpu.cc:308.
    """
    dt = q.dtype
    o, s = sdpa_fwd(q.astype(np.float32), k.astype(np.float32), v.astype(np.float32), **kw)
    return o.astype(dt), s


def sdpa_bwd_gate(q, k, v, o, stats, d_o, **kw):
    """Gating oracle for the backward: fp32 instantiation, all accumulation in fp32."""
    dt = q.dtype
    f = lambda a: a.astype(np.float32)
    dq, dk, dv = sdpa_bwd(f(q), f(k), f(v), f(o), stats, f(d_o), **kw)
    return dq.astype(dt), dk.astype(dt), dv.astype(dt)
