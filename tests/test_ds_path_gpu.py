"""The dS path of the backward: with the workspace of
sdpa_hip_bwd_workspace_bytes_ds, the dK/dV kernel stores the dS it forms and
dQ is one product with it (sdpa_f16_dq_ds.hip for fp16, sdpa_f32_dq_ds.hip
for fp32).

Every case is checked three ways:
  - against the oracle, at north_star's fp16 tolerances (run_and_check, which
    goes through pkg.sdpa_grad and so through the dS path);
  - against the path that forms dS in both kernels (the per-row workspace
    only): dK and dV bit-identical (same dK/dV kernel, and the row kernel
    hands it the values the other path's dQ kernel computes), dQ within the
    rounding of P to fp16 before dS is formed (fp16), or of the other path's
    own summation order for S and dP (fp32);
  - the three launches as separate calls (sdpa_hip_bwd_ds_phase) against the
    single call, bit-identical.
Shapes cover several key tiles, ragged query and key lengths (the last query
block and the last key group partial), cross attention both ways, both
128-wide sides, dropout, dropout > 1 (every element dropped) and one row."""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from _common import Cfg
from test_parity_gpu import _np, _t, run_and_check

pytestmark = pytest.mark.gpu

CASES = [
    Cfg("ds_causal_d128_p0.1", "f16", 3, 333, 333, 128, 128, True, 0.1, 128 ** -0.5, 5, 9),
    Cfg("ds_causal_d128_S1024", "f16", 4, 1024, 1024, 128, 128, True, 0.1, 128 ** -0.5, 7, 0),
    Cfg("ds_causal_d96", "f16", 2, 200, 200, 96, 96, True, 0.0, 96 ** -0.5, 1, 2),
    Cfg("ds_cross_128x64", "f16", 2, 130, 300, 128, 64, False, 0.2, 128 ** -0.5, 3, 4),
    Cfg("ds_cross_64x128", "f16", 2, 300, 100, 64, 128, False, 0.0, 64 ** -0.5, 3, 4),
    Cfg("ds_cross_d80_31x1000", "f16", 1, 31, 1000, 80, 80, False, 0.1, 80 ** -0.5, 11, 3),
    Cfg("ds_causal_d128_drop_all", "f16", 2, 160, 160, 128, 128, True, 1.5, 128 ** -0.5, 2, 6),
    Cfg("ds_causal_d128_one_row", "f16", 2, 1, 1, 128, 128, True, 0.0, 128 ** -0.5, 0, 0),
    # feature sizes that end inside a pair of 16-byte chunks (the row kernel's
    # lanes read chunks 2 ks + h: chunk 9 of D_v = 72 reads as zero)
    Cfg("ds_causal_120x72", "f16", 2, 257, 257, 120, 72, True, 0.1, 120 ** -0.5, 4, 5),
    # fp32 (the split dK/dV kernel's query blocks of 32)
    Cfg("ds32_causal_d128_p0.1", "f32", 2, 300, 300, 128, 128, True, 0.1, 128 ** -0.5, 5, 9),
    Cfg("ds32_cross_128x64", "f32", 2, 100, 1000, 128, 64, False, 0.0, 128 ** -0.5, 3, 4),
    Cfg("ds32_cross_64x128_p0.2", "f32", 2, 257, 130, 64, 128, False, 0.2, 64 ** -0.5, 1, 2),
    Cfg("ds32_causal_100x36", "f32", 2, 161, 161, 100, 36, True, 0.05, 100 ** -0.5, 7, 8),
    Cfg("ds32_causal_drop_all", "f32", 2, 96, 96, 128, 128, True, 1.5, 128 ** -0.5, 2, 6),
    # a 32-wide D_qk beside a 128-wide D_v: dQ from dS with a 32-feature K
    # tile (one copy per wave, no row swizzle)
    Cfg("ds_causal_32x128", "f16", 2, 190, 190, 32, 128, True, 0.1, 32 ** -0.5, 6, 1),
    Cfg("ds32_cross_32x128", "f32", 2, 75, 260, 32, 128, False, 0.1, 32 ** -0.5, 8, 2),
    # fp32 with a narrow V side (the split dK/dV kernel's <128, 32> instantiation)
    Cfg("ds32_cross_128x16", "f32", 2, 140, 333, 128, 16, False, 0.1, 128 ** -0.5, 9, 4),
    Cfg("ds32_causal_96x32", "f32", 2, 170, 170, 96, 32, True, 0.0, 96 ** -0.5, 10, 5),
]


def _dcode(c):
    return 1 if c.dtype == "f16" else 0


def _bits(a):
    return a.view(np.uint16 if a.dtype == np.float16 else np.uint32)


def _grads(pkg, c, q, k, v, o, s, d_o, ds_path):
    kw = dict(dropout=c.dropout, scale=c.scale, causal_mask=c.causal)
    g = pkg.sdpa_grad(q, k, v, o, s, d_o, c.seed, c.offset, ds_path=ds_path, **kw)
    torch.cuda.synchronize()
    return [_np(x) for x in g]


def _phases(pkg, c, q, k, v, o, s, d_o):
    L = pkg.library()
    B, S_q, D_qk = q.shape
    S_kv, D_v = k.shape[1], v.shape[2]
    ws_bytes = int(L.sdpa_hip_bwd_workspace_bytes_ds(_dcode(c), B, S_q, S_kv, D_qk, D_v, int(c.causal)))
    ws = torch.empty((ws_bytes,), dtype=torch.uint8, device=q.device)
    dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
    h = torch.cuda.current_stream().cuda_stream
    for phase in range(3):
        rc = L.sdpa_hip_bwd_ds_phase(phase, _dcode(c), q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(),
                                     s.data_ptr(), d_o.data_ptr(), dq.data_ptr(), dk.data_ptr(),
                                     dv.data_ptr(), ws.data_ptr(), ws_bytes, B, S_q, S_kv, D_qk, D_v,
                                     float(c.scale), float(c.dropout), int(c.causal), c.seed, c.offset, h)
        assert rc == 0, pkg.status_string(rc)
    torch.cuda.synchronize()
    return [_np(x) for x in (dq, dk, dv)]


@pytest.mark.parametrize("c", CASES, ids=[c.name for c in CASES])
def test_ds_path(pkg, O, c):
    L = pkg.library()
    rows = int(L.sdpa_hip_bwd_workspace_bytes(c.B, c.S_q))
    full = int(L.sdpa_hip_bwd_workspace_bytes_ds(_dcode(c), c.B, c.S_q, c.S_kv, c.D_qk, c.D_v, int(c.causal)))
    assert full > rows  # the shape takes the dS path
    run_and_check(pkg, O, c, fp32_sum_allowance=True)

    from _common import make_inputs
    qn, kn, vn, don = make_inputs(c)
    q, k, v, d_o = _t(qn), _t(kn), _t(vn), _t(don)
    o, s = pkg.sdpa(q, k, v, c.seed, c.offset, dropout=c.dropout, scale=c.scale, causal_mask=c.causal)
    torch.cuda.synchronize()
    dq_a, dk_a, dv_a = _grads(pkg, c, q, k, v, o, s, d_o, True)
    dq_b, dk_b, dv_b = _grads(pkg, c, q, k, v, o, s, d_o, False)
    dq_p, dk_p, dv_p = _phases(pkg, c, q, k, v, o, s, d_o)
    f = lambda a: a.astype(np.float32)
    ddq = float(np.abs(f(dq_a) - f(dq_b)).max()) if dq_a.size else 0.0
    print(f"[ds] {c.name}: dq ds-path vs recompute max|diff|={ddq:.3e}", flush=True)
    assert np.array_equal(_bits(dk_a), _bits(dk_b))
    assert np.array_equal(_bits(dv_a), _bits(dv_b))
    # fp16: the recompute path forms dS from fp32 P, the dS path from its fp16
    # copy: a relative 2^-11 on each term before dS is rounded to fp16 itself.
    # fp32: the same dS up to the two kernels' summation orders for S and dP.
    scale_g = max(1.0, float(np.abs(f(dq_b)).max()) if dq_b.size else 1.0)
    assert ddq <= (4e-3 if c.dtype == "f16" else 2e-5) * scale_g
    for a, b in ((dq_a, dq_p), (dk_a, dk_p), (dv_a, dv_p)):
        assert np.array_equal(_bits(a), _bits(b))


def test_ds_path_workspace_selects_path(pkg, O):
    """A workspace one byte short of the dS size runs the other path (same
    dK, dV bits; dQ as that path computes it) and the phase entry point
    refuses it."""
    c = CASES[0]
    from _common import make_inputs
    qn, kn, vn, don = make_inputs(c)
    q, k, v, d_o = _t(qn), _t(kn), _t(vn), _t(don)
    o, s = pkg.sdpa(q, k, v, c.seed, c.offset, dropout=c.dropout, scale=c.scale, causal_mask=c.causal)
    L = pkg.library()
    B, S_q, D_qk = q.shape
    S_kv, D_v = k.shape[1], v.shape[2]
    full = int(L.sdpa_hip_bwd_workspace_bytes_ds(1, B, S_q, S_kv, D_qk, D_v, int(c.causal)))
    ws = torch.empty((full,), dtype=torch.uint8, device=q.device)
    h = torch.cuda.current_stream().cuda_stream
    outs = {}
    for nbytes in (full, full - 1):
        dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
        rc = L.sdpa_hip_bwd(1, q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(), s.data_ptr(),
                            d_o.data_ptr(), dq.data_ptr(), dk.data_ptr(), dv.data_ptr(), ws.data_ptr(),
                            nbytes, B, S_q, S_kv, D_qk, D_v, float(c.scale), float(c.dropout),
                            int(c.causal), c.seed, c.offset, h)
        assert rc == 0
        torch.cuda.synchronize()
        outs[nbytes] = [_np(x) for x in (dq, dk, dv)]
    ref_b = _grads(pkg, c, q, k, v, o, s, d_o, False)
    ref_a = _grads(pkg, c, q, k, v, o, s, d_o, True)
    for got, ref in zip(outs[full - 1], ref_b):
        assert np.array_equal(got.view(np.uint16), ref.view(np.uint16))
    for got, ref in zip(outs[full], ref_a):
        assert np.array_equal(got.view(np.uint16), ref.view(np.uint16))
    rc = L.sdpa_hip_bwd_ds_phase(2, 1, q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(), s.data_ptr(),
                                 d_o.data_ptr(), q.data_ptr(), k.data_ptr(), v.data_ptr(), ws.data_ptr(),
                                 full - 1, B, S_q, S_kv, D_qk, D_v, float(c.scale), float(c.dropout),
                                 int(c.causal), c.seed, c.offset, h)
    assert rc == pkg.SDPA_ERR_DS_PATH


def _ds_layout(S_q, S_kv, causal):
    """(kt, qb) -> chunk index within a batch row, and chunks per row: the
    order the split dK/dV kernel visits them (kt-major, its q_begin)."""
    idx, n = {}, 0
    for kt in range((S_kv + 127) // 128):
        q_begin = (min(128 * kt, S_q) // 64) * 64 if causal else 0
        for qb in range(q_begin // 64, (S_q + 63) // 64):
            idx[(kt, qb)] = n
            n += 1
    return idx, n


def _perm():
    """Query of stored position j within a 32-query sub-tile."""
    return np.array([8 * ((j >> 2) & 3) + 4 * (j >> 4) + (j & 3) for j in range(32)])


# S = 200 ends in an 8-key partial step: the rows past S_kv within a
# transposed read are not the last ones of it
@pytest.mark.parametrize("shape", [(2, 200, 200, 96, 96, True), (1, 200, 200, 128, 128, True),
                                   (1, 160, 160, 128, 128, True), (1, 100, 260, 128, 64, False)],
                         ids=["causal_d96_S200", "causal_d128_S200", "causal_d128", "cross_128x64"])
def test_ds_stored_and_dq_product(pkg, O, shape):
    """The stored dS' against a float64 dS of the same inputs at every stored
    position (the P role's fp16 P and the fp16 store bound the difference),
    and phase 2's dQ against scale * (stored dS') K evaluated on the host."""
    B, S_q, S_kv, D_qk, D_v, causal = shape
    c = Cfg("ds_diag", "f16", B, S_q, S_kv, D_qk, D_v, causal, 0.0, D_qk ** -0.5, 4, 1)
    from _common import make_inputs
    qn, kn, vn, don = make_inputs(c)
    q, k, v, d_o = _t(qn), _t(kn), _t(vn), _t(don)
    o, s = pkg.sdpa(q, k, v, 4, 1, dropout=0.0, scale=c.scale, causal_mask=causal)
    L = pkg.library()
    rows = int(L.sdpa_hip_bwd_workspace_bytes(B, S_q))
    full = int(L.sdpa_hip_bwd_workspace_bytes_ds(1, B, S_q, S_kv, D_qk, D_v, int(causal)))
    ws = torch.zeros((full,), dtype=torch.uint8, device=q.device)
    dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
    h = torch.cuda.current_stream().cuda_stream
    for phase in range(3):
        rc = L.sdpa_hip_bwd_ds_phase(phase, 1, q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(),
                                     s.data_ptr(), d_o.data_ptr(), dq.data_ptr(), dk.data_ptr(), dv.data_ptr(),
                                     ws.data_ptr(), full, B, S_q, S_kv, D_qk, D_v, float(c.scale), 0.0,
                                     int(causal), 4, 1, h)
        assert rc == 0
    torch.cuda.synchronize()
    raw = ws[rows:].cpu().numpy().view(np.float16).astype(np.float64)
    idx, per_row = _ds_layout(S_q, S_kv, causal)
    assert raw.size == B * per_row * 8192
    # inside a 2 KB key group (1024 halves): position i of key r sits in
    # plane p = 2 j + h (h = i >> 4, j = (i >> 3) & 1), row r ^ 4 p, half i & 7
    r_, i_ = np.meshgrid(np.arange(32), np.arange(32), indexing="ij")
    p_ = 2 * ((i_ >> 3) & 1) + (i_ >> 4)
    gather = p_ * 256 + (r_ ^ (4 * p_)) * 8 + (i_ & 7)
    assert sorted(gather.ravel()) == list(range(1024))
    chunks = raw.reshape(B, per_row, 2, 4, 1024)[..., gather].reshape(B, per_row, 2, 128, 32)
    pi = _perm()
    # float64 reference dS = P (dP - delta), P gated at 1e-6
    f64 = lambda a: a.astype(np.float64)
    o_h, s_h = f64(_np(o)), f64(_np(s))
    S = c.scale * np.einsum("bid,bjd->bij", f64(qn), f64(kn))
    P = np.exp(S - s_h[..., None])
    if causal:
        P = np.where(np.tril(np.ones((S_q, S_kv), bool))[None], P, 0.0)
    P = np.where(P > 1e-6, P, 0.0)
    dP = np.einsum("bid,bjd->bij", f64(don), f64(vn))
    delta = np.einsum("bid,bid->bi", f64(don), o_h)
    dS = P * (dP - delta[..., None])
    stored = np.zeros((B, S_q, S_kv))
    seen = np.zeros((B, S_q, S_kv), bool)
    for (kt, qb), ci in idx.items():
        for t in range(2):
            q_idx = qb * 64 + 32 * t + pi
            for kw in range(4):
                kw0 = 128 * kt + 32 * kw
                qs = qb * 64 + 32 * t
                if not (kw0 < S_kv and qs < S_q and not (causal and qs + 31 < kw0)):
                    continue
                blk = chunks[:, ci, t, 32 * kw:32 * kw + 32, :]  # [B, key, position]
                for kk in range(32):
                    key = kw0 + kk
                    if key >= S_kv:
                        continue
                    ok = q_idx < S_q
                    stored[:, q_idx[ok], key] = blk[:, kk, ok]
                    seen[:, q_idx[ok], key] = True
    need = np.abs(dS) > 0
    assert seen[need].all(), "a nonzero dS was not stored"
    err_ds = float(np.abs(stored - dS)[seen].max())
    ref_ds = float(np.abs(dS).max())
    dq_host = c.scale * np.einsum("bij,bjd->bid", stored, f64(kn))
    err_dq = float(np.abs(f64(_np(dq)) - dq_host).max())
    print(f"[ds] {shape}: stored dS max|err|={err_ds:.3e} (max|dS|={ref_ds:.3e}); "
          f"dQ vs scale*dS_stored*K max|err|={err_dq:.3e}", flush=True)
    assert err_ds <= 2e-3 * max(1.0, ref_ds)
    assert err_dq <= 2e-3 * max(1.0, float(np.abs(dq_host).max()))


def _slot32(key, pos):
    """Byte offset of (key, query position) inside a stored fp32 key group of
    32 keys (csrc/sdpa_params.h, DsLayout32::slot32): quarter u = the store
    holding positions 16 h + 4 u .. + 3, half h, the key's 16-byte slot at
    key ^ (u + 4 h)."""
    u, h = (pos >> 2) & 3, pos >> 4
    return 1024 * u + 512 * h + 16 * (key ^ (u + 4 * h)) + 4 * (pos & 3)


def _ds32_gather():
    """[128 keys, 32 positions] float indices into a 16 KB fp32 chunk."""
    g = np.empty((128, 32), np.int64)
    for key in range(128):
        for pos in range(32):
            g[key, pos] = ((key // 32) * 4096 + _slot32(key % 32, pos)) // 4
    assert np.unique(g).size == 4096
    return g


def _ds_layout32(S_q, S_kv, causal):
    """(kt, qb) -> chunk index within a batch row, and chunks per row, for the
    fp32 split dK/dV kernel: key tiles of 128, query blocks of 32 (its
    q_begin), kt-major."""
    idx, n = {}, 0
    for kt in range((S_kv + 127) // 128):
        q_begin = (min(128 * kt, S_q) // 32) * 32 if causal else 0
        for qb in range(q_begin // 32, (S_q + 31) // 32):
            idx[(kt, qb)] = n
            n += 1
    return idx, n


@pytest.mark.parametrize("shape", [(1, 200, 200, 128, 128, True), (2, 100, 260, 128, 64, False),
                                   (1, 70, 70, 100, 36, True)],
                         ids=["f32_causal_d128_S200", "f32_cross_128x64", "f32_causal_100x36"])
def test_ds32_stored_and_dq_product(pkg, O, shape):
    """fp32: the stored dS against a float64 dS of the same inputs at every
    stored position (decoded through _slot32: each key group of 32 keys as
    four 1 KB stores of 16-byte slots), and phase 2's dQ against
    scale * (stored dS) K."""
    B, S_q, S_kv, D_qk, D_v, causal = shape
    c = Cfg("ds32_diag", "f32", B, S_q, S_kv, D_qk, D_v, causal, 0.0, D_qk ** -0.5, 4, 1)
    from _common import make_inputs
    qn, kn, vn, don = make_inputs(c)
    q, k, v, d_o = _t(qn), _t(kn), _t(vn), _t(don)
    o, s = pkg.sdpa(q, k, v, 4, 1, dropout=0.0, scale=c.scale, causal_mask=causal)
    L = pkg.library()
    rows = int(L.sdpa_hip_bwd_workspace_bytes(B, S_q))
    full = int(L.sdpa_hip_bwd_workspace_bytes_ds(0, B, S_q, S_kv, D_qk, D_v, int(causal)))
    ws = torch.zeros((full,), dtype=torch.uint8, device=q.device)
    dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
    h = torch.cuda.current_stream().cuda_stream
    for phase in range(3):
        rc = L.sdpa_hip_bwd_ds_phase(phase, 0, q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(),
                                     s.data_ptr(), d_o.data_ptr(), dq.data_ptr(), dk.data_ptr(), dv.data_ptr(),
                                     ws.data_ptr(), full, B, S_q, S_kv, D_qk, D_v, float(c.scale), 0.0,
                                     int(causal), 4, 1, h)
        assert rc == 0
    torch.cuda.synchronize()
    raw = ws[rows:].cpu().numpy().view(np.float32).astype(np.float64)
    idx, per_row = _ds_layout32(S_q, S_kv, causal)
    assert raw.size == B * per_row * 4096
    chunks = raw.reshape(B, per_row, 4096)[:, :, _ds32_gather()]  # [chunk][key][position]
    pi = _perm()
    f64 = lambda a: a.astype(np.float64)
    o_h, s_h = f64(_np(o)), f64(_np(s))
    S = c.scale * np.einsum("bid,bjd->bij", f64(qn), f64(kn))
    P = np.exp(S - s_h[..., None])
    if causal:
        P = np.where(np.tril(np.ones((S_q, S_kv), bool))[None], P, 0.0)
    P = np.where(P > 1e-6, P, 0.0)
    dP = np.einsum("bid,bjd->bij", f64(don), f64(vn))
    delta = np.einsum("bid,bid->bi", f64(don), o_h)
    dS = P * (dP - delta[..., None])
    stored = np.zeros((B, S_q, S_kv))
    seen = np.zeros((B, S_q, S_kv), bool)
    for (kt, qb), ci in idx.items():
        q_idx = qb * 32 + pi
        for kw in range(4):
            kw0 = 128 * kt + 32 * kw
            q0 = 32 * qb
            if not (kw0 < S_kv and q0 < S_q and not (causal and q0 + 31 < kw0)):
                continue
            blk = chunks[:, ci, 32 * kw:32 * kw + 32, :]  # [B, key, position]
            for kk in range(32):
                key = kw0 + kk
                if key >= S_kv:
                    assert not blk[:, kk, :].any(), "keys past S_kv are stored as zero"
                    continue
                ok = q_idx < S_q
                stored[:, q_idx[ok], key] = blk[:, kk, ok]
                seen[:, q_idx[ok], key] = True
    need = np.abs(dS) > 0
    assert seen[need].all(), "a nonzero dS was not stored"
    err_ds = float(np.abs(stored - dS)[seen].max())
    ref_ds = float(np.abs(dS).max())
    dq_host = c.scale * np.einsum("bij,bjd->bid", stored, f64(kn))
    err_dq = float(np.abs(f64(_np(dq)) - dq_host).max())
    print(f"[ds32] {shape}: stored dS max|err|={err_ds:.3e} (max|dS|={ref_ds:.3e}); "
          f"dQ vs scale*dS_stored*K max|err|={err_dq:.3e}", flush=True)
    assert err_ds <= 1e-5 * max(1.0, ref_ds)
    assert err_dq <= 1e-5 * max(1.0, float(np.abs(dq_host).max()))
