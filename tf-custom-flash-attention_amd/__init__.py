"""MI355X (gfx950) implementation of the Sdpa / SdpaGrad ops.

Host-side mirror of the reference's Python op interface
(``README.md:28-56``, ``test.py:12-30``): ``sdpa(q, k, v, seed, offset,
dropout=, scale=, causal_mask=)`` returns ``(o, stats)`` and ``sdpa_grad(q, k,
v, o, stats, d_o, seed, offset, dropout=, scale=, causal_mask=)`` returns
``(dq, dk, dv)``, with the reference's argument checks and messages
(``sdpa/sdpa_cpu.cc:37-69,116-168``).  The gradient wiring of
``@tf.RegisterGradient("Sdpa")`` -- op inputs/outputs/attrs in, ``dq, dk, dv``
out, no gradient for seed/offset -- is :class:`SdpaFunction`.

Tensors are torch tensors on the GPU (torch is only the device-memory and
stream plumbing here); all arithmetic runs in the hand-written HIP kernels of
``libsdpa_hip.so`` through the C ABI in ``include/sdpa_hip.h``.  There is no
CPU fallback: if the library is missing, every entry point raises.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libsdpa_hip.so")

DTYPE_F32 = 0
DTYPE_F16 = 1

# sdpa_status_t (include/sdpa_hip.h)
SDPA_OK = 0
SDPA_ERR_HIP = 23
SDPA_ERR_SCRATCH_LIMIT = 24
SDPA_ERR_DS_PATH = 25
_ARG_ERRORS = set(range(1, 23)) | {SDPA_ERR_SCRATCH_LIMIT, SDPA_ERR_DS_PATH}

_lib = None


class InvalidArgumentError(ValueError):
    """Raised where the reference op fails with errors::InvalidArgument."""


class InternalError(RuntimeError):
    """Raised where a launch fails (the reference aborts via TF_CHECK_OK)."""


def build(jobs: int = 4) -> str:
    """Compile libsdpa_hip.so in-tree for gfx950 (hipcc via the package Makefile)."""
    subprocess.run(["make", "-s", "-C", _HERE, f"-j{jobs}", "libsdpa_hip.so"], check=True)
    return LIB_PATH


def library():
    """Load libsdpa_hip.so (raises if it has not been built)."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(f"{LIB_PATH} is missing: run __graft_entry__.build() (the HIP "
                           "extension is required; there is no CPU fallback)")
    L = ctypes.CDLL(LIB_PATH)
    vp, i32, i64p = ctypes.c_void_p, ctypes.c_int, ctypes.POINTER(ctypes.c_int64)
    f32, u64, sz = ctypes.c_float, ctypes.c_uint64, ctypes.c_size_t
    L.sdpa_hip_status_string.restype = ctypes.c_char_p
    L.sdpa_hip_status_string.argtypes = [i32]
    L.sdpa_hip_last_hip_error.restype = i32
    L.sdpa_hip_last_hip_error.argtypes = []
    L.sdpa_hip_check_fwd.restype = i32
    L.sdpa_hip_check_fwd.argtypes = [i32, i64p, i32, i64p, i32, i64p, i32, i32, i32]
    L.sdpa_hip_check_bwd.restype = i32
    L.sdpa_hip_check_bwd.argtypes = [i32, i64p, i32, i64p, i32, i64p, i32, i64p, i32, i64p,
                                     i32, i64p, i32, i32, i32]
    L.sdpa_hip_fwd.restype = i32
    L.sdpa_hip_fwd.argtypes = [i32, vp, vp, vp, vp, vp, i32, i32, i32, i32, i32, f32, f32, i32,
                               u64, u64, vp]
    L.sdpa_hip_bwd_workspace_bytes.restype = sz
    L.sdpa_hip_bwd_workspace_bytes.argtypes = [i32, i32]
    L.sdpa_hip_bwd.restype = i32
    L.sdpa_hip_bwd.argtypes = [i32, vp, vp, vp, vp, vp, vp, vp, vp, vp, vp, sz, i32, i32, i32,
                               i32, i32, f32, f32, i32, u64, u64, vp]
    L.sdpa_hip_bwd_dq.restype = i32
    L.sdpa_hip_bwd_dq.argtypes = [i32, vp, vp, vp, vp, vp, vp, vp, vp, sz, i32, i32, i32, i32,
                                  i32, f32, f32, i32, u64, u64, vp]
    L.sdpa_hip_bwd_dkdv.restype = i32
    L.sdpa_hip_bwd_dkdv.argtypes = [i32, vp, vp, vp, vp, vp, vp, vp, vp, sz, i32, i32, i32, i32,
                                    i32, f32, f32, i32, u64, u64, vp]
    L.sdpa_hip_bwd_workspace_bytes_ds.restype = sz
    L.sdpa_hip_bwd_workspace_bytes_ds.argtypes = [i32] * 7
    L.sdpa_hip_bwd_ds_phase.restype = i32
    L.sdpa_hip_bwd_ds_phase.argtypes = [i32, i32, vp, vp, vp, vp, vp, vp, vp, vp, vp, vp, sz, i32, i32,
                                        i32, i32, i32, f32, f32, i32, u64, u64, vp]
    L.sdpa_hip_bwd_noalloc.restype = i32
    L.sdpa_hip_bwd_noalloc.argtypes = [i32, vp, vp, vp, vp, vp, vp, vp, vp, vp, i32, i32, i32,
                                       i32, i32, f32, f32, i32, u64, u64, vp]
    L.sdpa_hip_drop_threshold.restype = u64
    L.sdpa_hip_drop_threshold.argtypes = [f32]
    L.sdpa_hip_dropout_mask.restype = i32
    L.sdpa_hip_dropout_mask.argtypes = [vp, i32, i32, i32, f32, u64, u64, vp]
    _lib = L
    return L


def status_string(code: int) -> str:
    return library().sdpa_hip_status_string(int(code)).decode()


def _raise_for(code: int) -> None:
    if code == SDPA_OK:
        return
    msg = status_string(code)
    if code == SDPA_ERR_HIP:
        raise InternalError(f"{msg} (hipError_t {library().sdpa_hip_last_hip_error()})")
    raise InvalidArgumentError(msg)


def _shape(x):
    import torch
    if isinstance(x, torch.Tensor):
        return tuple(int(d) for d in x.shape)
    return ()  # python int: a scalar


def _dims(shape):
    arr = (ctypes.c_int64 * max(1, len(shape)))(*shape)
    return len(shape), arr


def _u64(x) -> int:
    """Scalar seed/offset as uint64 (the reference reads scalar<uint64>)."""
    import torch
    if isinstance(x, torch.Tensor):
        x = int(x.item())
    return int(x) & 0xFFFFFFFFFFFFFFFF


def _dtype_code(t) -> int:
    import torch
    if t.dtype == torch.float16:
        return DTYPE_F16
    if t.dtype == torch.float32:
        return DTYPE_F32
    raise InvalidArgumentError(f"T must be half or float, got {t.dtype}")


def _stream_handle(device) -> int:
    import torch
    return torch.cuda.current_stream(device).cuda_stream


def _require_gpu(*ts) -> None:
    for t in ts:
        if not t.is_cuda:
            raise InvalidArgumentError("tensors must be on the GPU (the op's HIP kernel)")


def check_fwd(q, k, v, seed=0, offset=0, causal_mask=False) -> None:
    """Shape/validation checks of Sdpa (sdpa_ops.cc:22-25, sdpa_cpu.cc:37-69)."""
    rq, aq = _dims(_shape(q))
    rk, ak = _dims(_shape(k))
    rv, av = _dims(_shape(v))
    _raise_for(library().sdpa_hip_check_fwd(rq, aq, rk, ak, rv, av, len(_shape(seed)),
                                            len(_shape(offset)), int(bool(causal_mask))))


def check_bwd(q, k, v, o, stats, d_o, seed=0, offset=0, causal_mask=False) -> None:
    """Validation of SdpaGrad (sdpa_ops.cc:55-57, sdpa_cpu.cc:116-168)."""
    dims = [_dims(_shape(t)) for t in (q, k, v, o, stats, d_o)]
    flat = [x for d in dims for x in d]
    _raise_for(library().sdpa_hip_check_bwd(*flat, len(_shape(seed)), len(_shape(offset)),
                                            int(bool(causal_mask))))


def sdpa(q, k, v, seed=0, offset=0, dropout: float = 0.0, scale: float = 1.0,
         causal_mask: bool = False):
    """Forward op ``Sdpa`` (sdpa_ops.cc:7-32): returns ``(o, stats)``.

    q [B,S_q,D_qk], k [B,S_kv,D_qk], v [B,S_kv,D_v] (fp16 or fp32, same dtype);
    o [B,S_q,D_v] in that dtype, stats [B,S_q] fp32.
    """
    import torch
    check_fwd(q, k, v, seed, offset, causal_mask)
    if not (q.dtype == k.dtype == v.dtype):
        raise InvalidArgumentError("q, k and v must have the same dtype T")
    dt = _dtype_code(q)
    _require_gpu(q, k, v)
    q, k, v = q.contiguous(), k.contiguous(), v.contiguous()
    B, S_q, D_qk = q.shape
    S_kv, D_v = k.shape[1], v.shape[2]
    o = torch.empty((B, S_q, D_v), dtype=q.dtype, device=q.device)
    stats = torch.empty((B, S_q), dtype=torch.float32, device=q.device)
    rc = library().sdpa_hip_fwd(dt, q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(),
                                stats.data_ptr(), B, S_q, S_kv, D_qk, D_v, float(scale),
                                float(dropout), int(bool(causal_mask)), _u64(seed), _u64(offset),
                                _stream_handle(q.device))
    _raise_for(rc)
    return o, stats


def sdpa_grad(q, k, v, o, stats, d_o, seed=0, offset=0, dropout: float = 0.0,
              scale: float = 1.0, causal_mask: bool = False, *, ds_path: bool = True):
    """Gradient op ``SdpaGrad`` (sdpa_ops.cc:34-63): returns ``(dq, dk, dv)``.

    ``ds_path``: give the backward the workspace of its dS path
    (``sdpa_hip_bwd_workspace_bytes_ds``: float16 or float32 with a feature
    size over 64 then stores dS in the dK/dV kernel and forms dQ from it); False gives
    it the per-row workspace only, and both kernels form dS."""
    import torch
    check_bwd(q, k, v, o, stats, d_o, seed, offset, causal_mask)
    if not (q.dtype == k.dtype == v.dtype == o.dtype == d_o.dtype):
        raise InvalidArgumentError("q, k, v, out and do must have the same dtype T")
    if stats.dtype != torch.float32:
        raise InvalidArgumentError("stats must be float32")
    dt = _dtype_code(q)
    _require_gpu(q, k, v, o, stats, d_o)
    q, k, v, o, stats, d_o = (t.contiguous() for t in (q, k, v, o, stats, d_o))
    B, S_q, D_qk = q.shape
    S_kv, D_v = k.shape[1], v.shape[2]
    L = library()
    dq = torch.empty_like(q)
    dk = torch.empty_like(k)
    dv = torch.empty_like(v)
    if ds_path:
        ws_bytes = int(L.sdpa_hip_bwd_workspace_bytes_ds(dt, B, S_q, S_kv, D_qk, D_v,
                                                         int(bool(causal_mask))))
    else:
        ws_bytes = int(L.sdpa_hip_bwd_workspace_bytes(B, S_q))
    ws = torch.empty((max(ws_bytes, 1),), dtype=torch.uint8, device=q.device)
    rc = L.sdpa_hip_bwd(dt, q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(),
                        stats.data_ptr(), d_o.data_ptr(), dq.data_ptr(), dk.data_ptr(),
                        dv.data_ptr(), ws.data_ptr(), ws_bytes, B, S_q, S_kv, D_qk, D_v,
                        float(scale), float(dropout), int(bool(causal_mask)), _u64(seed),
                        _u64(offset), _stream_handle(q.device))
    _raise_for(rc)
    return dq, dk, dv


def drop_threshold(dropout: float) -> int:
    """T(p): the element is dropped iff (hash >> 32) < T(p)."""
    return int(library().sdpa_hip_drop_threshold(float(dropout)))


def dropout_keep_mask(B: int, S_q: int, S_kv: int, dropout: float, seed=0, offset=0,
                      device="cuda"):
    """uint8 [B,S_q,S_kv] keep mask computed on the device by the kernels' hash."""
    import torch
    keep = torch.empty((B, S_q, S_kv), dtype=torch.uint8, device=device)
    rc = library().sdpa_hip_dropout_mask(keep.data_ptr(), B, S_q, S_kv, float(dropout), _u64(seed),
                                         _u64(offset), _stream_handle(keep.device))
    _raise_for(rc)
    return keep


def _make_function():
    import torch

    class SdpaFunction(torch.autograd.Function):
        """``Sdpa`` with its registered gradient (reference ``_sdpa_grad``,
        test.py:19-30): backward calls ``sdpa_grad`` with the op's inputs,
        outputs and attrs and returns ``dq, dk, dv`` and no gradient for
        seed/offset."""

        @staticmethod
        def forward(ctx, q, k, v, seed, offset, dropout, scale, causal_mask):
            o, s = sdpa(q, k, v, seed, offset, dropout=dropout, scale=scale,
                        causal_mask=causal_mask)
            ctx.save_for_backward(q, k, v, o, s)
            ctx.attrs = (seed, offset, dropout, scale, causal_mask)
            ctx.mark_non_differentiable(s)
            return o, s

        @staticmethod
        def backward(ctx, d_o, _d_s):
            q, k, v, o, s = ctx.saved_tensors
            seed, offset, dropout, scale, causal_mask = ctx.attrs
            dq, dk, dv = sdpa_grad(q, k, v, o, s, d_o.contiguous(), seed, offset,
                                   dropout=dropout, scale=scale, causal_mask=causal_mask)
            return dq, dk, dv, None, None, None, None, None

    return SdpaFunction


_fn = None


def sdpa_autograd(q, k, v, seed=0, offset=0, dropout: float = 0.0, scale: float = 1.0,
                  causal_mask: bool = False):
    """Differentiable ``sdpa``: ``(o, stats)`` with the SdpaGrad backward attached."""
    global _fn
    if _fn is None:
        _fn = _make_function()
    return _fn.apply(q, k, v, seed, offset, dropout, scale, causal_mask)
