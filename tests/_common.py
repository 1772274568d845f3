"""Shared helpers for the parity tests: the five BASELINE configurations,
seeded inputs, tolerances and the gating oracle wrappers."""
from __future__ import annotations

import math
from dataclasses import dataclass, field

import numpy as np


@dataclass
class Cfg:
    name: str
    dtype: str           # "f32" | "f16"
    B: int
    S_q: int
    S_kv: int
    D_qk: int
    D_v: int
    causal: bool
    dropout: float
    scale: float
    seed: int = 0
    offset: int = 0
    v_dist: str = "normal"     # "normal" | "uniform"  (c5: v ~ U(-1,1))
    do_kind: str = "normal"    # "normal" | "argmax"   (c1/c2: loss = sum(reduce_max(o,-1)))
    check_batches: tuple = field(default=())  # batch subset checked against the oracle ((): all)


# BASELINE.json "configs", in order.
CONFIGS = [
    Cfg("c1_f32_ref", "f32", 20, 400, 400, 32, 4, False, 0.0, 1 / math.sqrt(32), do_kind="argmax"),
    Cfg("c2_f16_dropout", "f16", 20, 400, 400, 32, 4, False, 0.2, 1 / math.sqrt(32), 42, 1000,
        do_kind="argmax"),
    Cfg("c3_f16_mha_causal", "f16", 256, 2048, 2048, 64, 64, True, 0.0, 1 / 8,
        check_batches=(0, 97, 255)),
    Cfg("c4_f16_headline", "f16", 128, 4096, 4096, 128, 128, True, 0.1, 1 / math.sqrt(128), 7, 0,
        check_batches=(0, 127)),
    Cfg("c5_f32_cross", "f32", 64, 512, 16384, 128, 64, False, 0.0, 1 / math.sqrt(128),
        v_dist="uniform", check_batches=(0, 63)),
]

TOL = {
    # north_star: fp32 within 1e-5 max-abs; fp16 2e-3 on o and 1e-2 on gradients.
    "f32": {"o": 1e-5, "grad": 1e-5, "stats": 1e-5},
    "f16": {"o": 2e-3, "grad": 1e-2, "stats": 1e-3},
}


def np_dtype(dt: str):
    return np.float16 if dt == "f16" else np.float32


def make_inputs(c: Cfg, seeds=(1024, 124, 24, 4)):
    """q, k, v (and dO ~ N(0,1)) from numpy PCG64, one seed per tensor; fp16
    values are drawn in fp32 and rounded to nearest even."""
    dt = np_dtype(c.dtype)
    gq, gk, gv, gd = (np.random.Generator(np.random.PCG64(s)) for s in seeds)
    q = gq.standard_normal((c.B, c.S_q, c.D_qk), dtype=np.float32).astype(dt)
    k = gk.standard_normal((c.B, c.S_kv, c.D_qk), dtype=np.float32).astype(dt)
    if c.v_dist == "uniform":
        v = gv.uniform(-1, 1, (c.B, c.S_kv, c.D_v)).astype(np.float32).astype(dt)
    else:
        v = gv.standard_normal((c.B, c.S_kv, c.D_v), dtype=np.float32).astype(dt)
    d_o = gd.standard_normal((c.B, c.S_q, c.D_v), dtype=np.float32).astype(dt)
    return q, k, v, d_o


def argmax_grad(o: np.ndarray) -> np.ndarray:
    """dO of loss = sum(reduce_max(o, -1)) (test.py:98): one-hot at each row's
    maximum, split equally among ties as TF's reduce_max gradient does."""
    of = o.astype(np.float32)
    m = of.max(axis=-1, keepdims=True)
    hit = (of == m).astype(np.float32)
    return (hit / hit.sum(axis=-1, keepdims=True)).astype(o.dtype)


def sub_batches(a: np.ndarray, batches) -> np.ndarray:
    return a if not batches else a[list(batches)]


def oracle_kw(c: Cfg, b0: int = 0):
    """Keyword arguments of the oracle for a run whose first batch is global
    batch b0: the dropout counter is linear in the batch index, so a batch
    subset is checked with offset + b0 * S_q * S_kv."""
    return dict(scale=c.scale, dropout=c.dropout, causal_mask=c.causal, seed=c.seed,
                offset=(c.offset + b0 * c.S_q * c.S_kv) & 0xFFFFFFFFFFFFFFFF)


def maxabs(a, b) -> float:
    if a.size == 0:
        return 0.0
    return float(np.abs(a.astype(np.float64) - b.astype(np.float64)).max())


def fwd_flops(c: Cfg) -> float:
    return 2.0 * c.B * c.S_q * c.S_kv * (c.D_qk + c.D_v) * (0.5 if c.causal else 1.0)


def bwd_flops(c: Cfg) -> float:
    return 2.0 * c.B * c.S_q * c.S_kv * (3 * c.D_qk + 2 * c.D_v) * (0.5 if c.causal else 1.0)
