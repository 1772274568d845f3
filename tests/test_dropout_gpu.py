"""Bit-exact dropout masks (north_star: "dropout masks must match bit-exactly").

The reference drops element (b, i, j) iff u(b, i, j) < p with u from the LCG
counter hash of sdpa/sdpa_utils.cuh:13-19 (= sdpa/sdpa_cpu.cc:198-211).  The
mask depends only on (b, i, j, S_q, S_kv, seed + offset), never on the
values, so it is read back through each production kernel with selector
inputs (q = 0 makes P uniform; one-hot V / dO / K expose single columns):

  forward : V[j, d] = [j == d + 128 t]        ->  o[b, i, d]  > 0  iff kept(i, d + 128 t)
  dK/dV   : dO[i, d] = [i == d + 128 t]       ->  dV[b, j, d] > 0  iff kept(d + 128 t, j)
  dQ      : K[j, d] = [j == d + 128 t], V = dO = e_0
            dS(i, j) = P * (keep * dP/(1-p) - delta_i) with dP = 1 > delta_i * (1-p)
                                              ->  dQ[b, i, d] > 0  iff kept(i, d + 128 t)
Each is compared bit-for-bit with the oracle's mask (the reference's float
predicate u < p evaluated on the CPU)."""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu
DEV = "cuda:0"

# (B, S_q, S_kv, p, seed, offset, dtype): c2's shape and key, a causal shape of
# the headline key, and tails that are not multiples of any tile size.
MASK_CASES = [
    (20, 400, 400, 0.2, 42, 1000, torch.float16),
    (2, 300, 300, 0.1, 7, 0, torch.float16),
    (3, 130, 257, 0.5, 123456789, 2**63 + 17, torch.float16),
    (2, 200, 144, 0.3, 5, 6, torch.float32),
]


def _ids(c):
    return f"B{c[0]}_{c[1]}x{c[2]}_p{c[3]}_{'f16' if c[6] == torch.float16 else 'f32'}"


@pytest.mark.parametrize("case", MASK_CASES, ids=[_ids(c) for c in MASK_CASES])
def test_device_mask_dump(pkg, O, case):
    B, S_q, S_kv, p, seed, off, _ = case
    got = pkg.dropout_keep_mask(B, S_q, S_kv, p, seed, off).cpu().numpy()
    ref = O.keep_mask(B, S_q, S_kv, p, seed, off)
    assert np.array_equal(got, ref), int((got != ref).sum())


@pytest.mark.parametrize("case", MASK_CASES, ids=[_ids(c) for c in MASK_CASES])
def test_forward_kernel_mask(pkg, O, case):
    B, S_q, S_kv, p, seed, off, dt = case
    ref = O.keep_mask(B, S_q, S_kv, p, seed, off)
    q = torch.zeros((B, S_q, 16), dtype=dt, device=DEV)
    k = torch.randn((B, S_kv, 16), device=DEV).to(dt)
    got = np.zeros_like(ref)
    for t in range((S_kv + 127) // 128):
        v = torch.zeros((B, S_kv, 128), dtype=dt, device=DEV)
        j = torch.arange(128 * t, min(S_kv, 128 * t + 128), device=DEV)
        v[:, j, j - 128 * t] = 1
        o, _ = pkg.sdpa(q, k, v, seed, off, dropout=p, scale=1.0, causal_mask=False)
        got[:, :, 128 * t:128 * t + len(j)] = (o[:, :, :len(j)] > 0).cpu().numpy()
    assert np.array_equal(got, ref), int((got != ref).sum())


@pytest.mark.parametrize("case", MASK_CASES, ids=[_ids(c) for c in MASK_CASES])
def test_dkdv_kernel_mask(pkg, O, case):
    B, S_q, S_kv, p, seed, off, dt = case
    ref = O.keep_mask(B, S_q, S_kv, p, seed, off)
    q = torch.zeros((B, S_q, 16), dtype=dt, device=DEV)
    k = torch.randn((B, S_kv, 16), device=DEV).to(dt)
    v = torch.randn((B, S_kv, 128), device=DEV).to(dt)
    o, s = pkg.sdpa(q, k, v, seed, off, dropout=p, scale=1.0)
    got = np.zeros_like(ref)
    for t in range((S_q + 127) // 128):
        d_o = torch.zeros((B, S_q, 128), dtype=dt, device=DEV)
        i = torch.arange(128 * t, min(S_q, 128 * t + 128), device=DEV)
        d_o[:, i, i - 128 * t] = 1
        _, _, dv = pkg.sdpa_grad(q, k, v, o, s, d_o, seed, off, dropout=p, scale=1.0)
        # dv[b, j, d] > 0 iff row i = d + 128 t keeps key j
        got[:, 128 * t:128 * t + len(i), :] = (dv[:, :, :len(i)] > 0).permute(0, 2, 1).cpu().numpy()
    assert np.array_equal(got, ref), int((got != ref).sum())


@pytest.mark.parametrize("case", MASK_CASES, ids=[_ids(c) for c in MASK_CASES])
def test_dq_kernel_mask(pkg, O, case):
    B, S_q, S_kv, p, seed, off, dt = case
    ref = O.keep_mask(B, S_q, S_kv, p, seed, off)
    q = torch.zeros((B, S_q, 128), dtype=dt, device=DEV)
    v = torch.zeros((B, S_kv, 8), dtype=dt, device=DEV)
    v[:, :, 0] = 1
    d_o = torch.zeros((B, S_q, 8), dtype=dt, device=DEV)
    d_o[:, :, 0] = 1
    got = np.zeros_like(ref)
    for t in range((S_kv + 127) // 128):
        k = torch.zeros((B, S_kv, 128), dtype=dt, device=DEV)
        j = torch.arange(128 * t, min(S_kv, 128 * t + 128), device=DEV)
        k[:, j, j - 128 * t] = 1
        o, s = pkg.sdpa(q, k, v, seed, off, dropout=p, scale=1.0)
        dq, _, _ = pkg.sdpa_grad(q, k, v, o, s, d_o, seed, off, dropout=p, scale=1.0)
        got[:, :, 128 * t:128 * t + len(j)] = (dq[:, :, :len(j)] > 0).cpu().numpy()
    assert np.array_equal(got, ref), int((got != ref).sum())


def test_headline_key_batch_subset(pkg, O):
    """Headline key (seed 7, offset 0, p 0.1, S 4096) on the batches 0 and 127
    of B = 128 via the linear counter: batch b of the full run equals batch 0
    of a run with offset + b * S^2."""
    S, p = 4096, 0.1
    for b in (0, 127):
        off = b * S * S
        got = pkg.dropout_keep_mask(1, S, S, p, 7, off).cpu().numpy()
        ref = O.keep_mask(1, S, S, p, 7, off)
        assert np.array_equal(got, ref)
        # drop rate close to p on 16.7M samples
        assert abs(1.0 - got.mean() - p) < 1e-3


# ---------------------------------------------------------------------------
# Causal runs at the DMA kernels' own widths (D_qk = D_v = D): the masked
# diagonal sub-tiles and the causal branches of every kernel apply the hash.
# ---------------------------------------------------------------------------
def _masks_through_kernels(pkg, B, S, p, seed, off, D, causal=True, dt=torch.float16):
    """(forward, dK/dV, dQ) keep masks read back through the production
    kernels at width D; entries the causal mask hides read as 0.

      forward : q = 0, V[j, d] = [j == d + D t]          -> o[i, d] > 0
      dK/dV   : q = 0, dO[i, d] = [i == d + D t]         -> dV[j, d] > 0
      dQ      : q = 0, K[j, d] = [j == d + D t], V = dO = e_0, and O = 0
                passed to the backward, so delta = 0 and
                dS(i, j) = P keep / (1 - p) > 0 exactly for kept elements
                                                          -> dQ[i, d] > 0
    (with the real O, a row whose elements are all kept has dS = 0 for every
    element, which a causal row 0 often is)."""
    shape = (B, S, D)
    zeros = lambda: torch.zeros(shape, dtype=dt, device=DEV)
    kw = dict(dropout=p, scale=1.0, causal_mask=causal)
    q = zeros()
    k_rand = torch.randn(shape, device=DEV).to(dt)
    v_rand = torch.randn(shape, device=DEV).to(dt)
    fwd = np.zeros((B, S, S), np.uint8)
    dkdv = np.zeros_like(fwd)
    dq = np.zeros_like(fwd)
    o_r, s_r = pkg.sdpa(q, k_rand, v_rand, seed, off, **kw)
    e0 = zeros()
    e0[:, :, 0] = 1
    for t in range((S + D - 1) // D):
        idx = torch.arange(D * t, min(S, D * t + D), device=DEV)
        n = len(idx)
        onehot = zeros()
        onehot[:, idx, idx - D * t] = 1
        o, _ = pkg.sdpa(q, k_rand, onehot, seed, off, **kw)
        fwd[:, :, D * t:D * t + n] = (o[:, :, :n] > 0).cpu().numpy()
        _, _, dv = pkg.sdpa_grad(q, k_rand, v_rand, o_r, s_r, onehot, seed, off, **kw)
        dkdv[:, D * t:D * t + n, :] = (dv[:, :, :n] > 0).permute(0, 2, 1).cpu().numpy()
        _, s1 = pkg.sdpa(q, onehot, e0, seed, off, **kw)
        g, _, _ = pkg.sdpa_grad(q, onehot, e0, zeros(), s1, e0, seed, off, **kw)
        dq[:, :, D * t:D * t + n] = (g[:, :, :n] > 0).cpu().numpy()
    torch.cuda.synchronize()
    return fwd, dkdv, dq


def _expected(O, B, S, p, seed, off, causal=True):
    ref = O.keep_mask(B, S, S, p, seed, off)
    if causal:
        ref &= np.tril(np.ones((S, S), np.uint8))[None]
    return ref


CAUSAL_CASES = [
    # (B, S, p, seed, offset, D)
    (2, 300, 0.1, 7, 0, 128),
    (2, 300, 0.2, 42, 1000, 64),
    (1, 333, 0.5, 99, 2**40 + 3, 128),
    (3, 200, 0.3, 5, 6, 32),
    (2, 130, 0.25, 11, 12, 64),
]


@pytest.mark.parametrize("case", CAUSAL_CASES, ids=[f"B{c[0]}_S{c[1]}_p{c[2]}_D{c[5]}" for c in CAUSAL_CASES])
def test_causal_masks_through_kernels(pkg, O, case):
    B, S, p, seed, off, D = case
    print(f"[case] causal mask B={B} S={S} p={p} D={D}", flush=True)
    ref = _expected(O, B, S, p, seed, off)
    for name, got in zip(("fwd", "dkdv", "dq"), _masks_through_kernels(pkg, B, S, p, seed, off, D)):
        assert np.array_equal(got, ref), (name, int((got != ref).sum()))


@pytest.mark.parametrize("b", [0, 127])
def test_headline_masks_through_kernels(pkg, O, b):
    """c4's own instantiation (fp16, D_qk = D_v = 128, causal, p = 0.1,
    seed 7, S = 4096) for batches 0 and 127 of B = 128: batch b of the full
    run is batch 0 of a run with offset + b S^2 (the counter is linear)."""
    S, p, seed = 4096, 0.1, 7
    off = b * S * S
    print(f"[case] headline mask batch {b}", flush=True)
    ref = _expected(O, 1, S, p, seed, off)
    for name, got in zip(("fwd", "dkdv", "dq"), _masks_through_kernels(pkg, 1, S, p, seed, off, 128)):
        assert np.array_equal(got, ref), (name, int((got != ref).sum()))
