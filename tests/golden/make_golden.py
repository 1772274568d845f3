"""Writes the golden fixtures of tests/golden/ (run: python tests/golden/make_golden.py).

Nothing here imports or runs the reference: the fixtures come from code of
this repository that is independent of the C++ oracle under oracle/:

* rng_known_answers.json -- the dropout hash restated in Python integers
  from its three agreeing statements in the reference (sdpa/sdpa_utils.cuh:13-19,
  sdpa/sdpa_cpu.cc:198-211, test.py:33-46): 64-bit words, u and the drop
  decision for p in {0.1, 0.2, 0.5} at the BASELINE keys.
* tiny_attention.npz -- float64 dense attention in the form of the
  reference's own dense check (test.py:65-88: scores in fp, causal -1e9
  mask, softmax, element-wise dropout mask from the hash, P V), extended with
  the reference op's two epsilons (stats = m + log(l + 1e-6), sdpa_cpu.cc:302)
  and the closed-form gradients, on tiny shapes with and without causal
  masking and dropout.  Arrays only (loaded with allow_pickle=False).
"""
from __future__ import annotations

import json
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
M64 = (1 << 64) - 1


def rng_bits(seed, offset, b, i, j, S_q, S_kv):
    idx = b * S_q * S_kv + i * S_kv + j
    state = (int(seed) + int(offset) + idx) & M64
    state = (state * 6364136223846793005 + 1442695040888963407) & M64
    return state >> 32


def rng_uniform(val):
    return float(np.float32(val) / np.float32(4294967296.0))


def keep_mask(B, S_q, S_kv, p, seed, offset):
    keep = np.ones((B, S_q, S_kv), dtype=np.uint8)
    if not p > 0:
        return keep
    for b in range(B):
        for i in range(S_q):
            for j in range(S_kv):
                if rng_uniform(rng_bits(seed, offset, b, i, j, S_q, S_kv)) < np.float32(p):
                    keep[b, i, j] = 0
    return keep


def dense_forward(q, k, v, scale, causal, p, keep):
    """float64; returns o, stats, P (undropped softmax), Pd (dropped, rescaled)."""
    s = scale * np.einsum("bid,bjd->bij", q, k)
    if causal:
        S_q, S_kv = s.shape[1:]
        mask = np.arange(S_kv)[None, :] > np.arange(S_q)[:, None]
        s = np.where(mask[None], -np.inf, s)
    m = s.max(-1, keepdims=True)
    e = np.exp(s - m)
    l = e.sum(-1, keepdims=True)
    stats = (m + np.log(l + 1e-6))[..., 0]
    P = e / l
    Pd = P * keep / (1.0 - p) if p > 0 else P
    o = np.einsum("bij,bjd->bid", Pd, v)
    return o, stats, P, Pd


def dense_backward(q, k, v, o, d_o, scale, p, keep, P, Pd):
    """Closed-form gradients of o = (softmax(scale q k^T) * keep / (1-p)) v."""
    dPd = np.einsum("bid,bjd->bij", d_o, v)
    dP = dPd * keep / (1.0 - p) if p > 0 else dPd
    delta = (d_o * o).sum(-1, keepdims=True)
    dS = P * (dP - delta)
    dq = scale * np.einsum("bij,bjd->bid", dS, k)
    dk = scale * np.einsum("bij,bid->bjd", dS, q)
    dv = np.einsum("bij,bid->bjd", Pd, d_o)
    return dq, dk, dv


TINY = [
    # name, B, S_q, S_kv, D_qk, D_v, causal, p, seed, offset
    ("plain", 2, 5, 7, 4, 3, False, 0.0, 0, 0),
    ("causal", 2, 6, 6, 5, 4, True, 0.0, 0, 0),
    ("dropout", 2, 5, 9, 4, 6, False, 0.2, 42, 1000),
    ("causal_dropout", 3, 7, 7, 8, 8, True, 0.5, 7, 3),
]


def main():
    answers = []
    keys = [(42, 1000, 400, 400, [(0, 0, 0), (0, 0, 1), (0, 1, 0), (19, 399, 399), (7, 123, 321)]),
            (7, 0, 4096, 4096, [(0, 0, 0), (127, 4095, 4095), (5, 1000, 17), (64, 2048, 4095)]),
            (2**64 - 5, 11, 3, 5, [(0, 0, 0), (2, 4, 4)])]
    for seed, off, S_q, S_kv, pts in keys:
        for b, i, j in pts:
            val = rng_bits(seed, off, b, i, j, S_q, S_kv)
            u = rng_uniform(val)
            answers.append(dict(seed=seed, offset=off, b=b, i=i, j=j, S_q=S_q, S_kv=S_kv,
                                bits=val, u=u, dropped={str(p): bool(u < np.float32(p))
                                                        for p in (0.1, 0.2, 0.5)}))
    with open(os.path.join(HERE, "rng_known_answers.json"), "w") as f:
        json.dump(answers, f, indent=1)

    arrays = {}
    rng = np.random.Generator(np.random.PCG64(2024))
    for name, B, S_q, S_kv, D_qk, D_v, causal, p, seed, off in TINY:
        q = rng.standard_normal((B, S_q, D_qk)).astype(np.float32)
        k = rng.standard_normal((B, S_kv, D_qk)).astype(np.float32)
        v = rng.standard_normal((B, S_kv, D_v)).astype(np.float32)
        d_o = rng.standard_normal((B, S_q, D_v)).astype(np.float32)
        scale = 1.0 / np.sqrt(D_qk)
        keep = keep_mask(B, S_q, S_kv, p, seed, off)
        o, stats, P, Pd = dense_forward(q.astype(np.float64), k.astype(np.float64),
                                        v.astype(np.float64), scale, causal, p, keep)
        dq, dk, dv = dense_backward(q.astype(np.float64), k.astype(np.float64),
                                    v.astype(np.float64), o, d_o.astype(np.float64), scale, p,
                                    keep, P, Pd)
        meta = np.array([B, S_q, S_kv, D_qk, D_v, int(causal), seed, off], dtype=np.uint64)
        for key, val in dict(q=q, k=k, v=v, d_o=d_o, keep=keep, o=o, stats=stats, dq=dq, dk=dk,
                             dv=dv, meta=meta, p=np.array([p, scale])).items():
            arrays[f"{name}__{key}"] = val
    np.savez(os.path.join(HERE, "tiny_attention.npz"), **arrays)


if __name__ == "__main__":
    main()
