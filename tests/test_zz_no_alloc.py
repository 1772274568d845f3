"""sdpa_hip_bwd_noalloc (the backward that allocates nothing; its per-row
values live in a static device array) against sdpa_hip_bwd with a
caller-allocated workspace, through the C ABI: identical kernels and inputs,
so dQ, dK and dV must agree bit for bit.  Two calls in a row, the second on
a smaller problem (the array keeps the first call's contents), then a size
beyond the array's limit, rejected before any device work."""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu
DEV = "cuda:0"

CASES = [
    # dtype, B, S_q, S_kv, D_qk, D_v, causal, dropout, seed, offset
    (torch.float16, 8, 1024, 1024, 128, 128, True, 0.1, 7, 0),
    (torch.float16, 2, 300, 200, 64, 32, False, 0.2, 42, 1000),
    (torch.float32, 3, 130, 130, 64, 64, True, 0.0, 1, 2),
]


def _run(pkg, case, noalloc):
    dt, B, S_q, S_kv, D_qk, D_v, causal, p, seed, off = case
    L = pkg.library()
    g = torch.Generator(device=DEV)
    g.manual_seed(B * 1000 + S_q)
    rnd = lambda *s: torch.randn(s, generator=g, device=DEV, dtype=torch.float32).to(dt)
    q, k, v = rnd(B, S_q, D_qk), rnd(B, S_kv, D_qk), rnd(B, S_kv, D_v)
    d_o = rnd(B, S_q, D_v)
    scale = D_qk ** -0.5
    o, s = pkg.sdpa(q, k, v, seed, off, dropout=p, scale=scale, causal_mask=causal)
    dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
    dcode = pkg.DTYPE_F16 if dt == torch.float16 else pkg.DTYPE_F32
    h = torch.cuda.current_stream(DEV).cuda_stream
    args = (q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(), s.data_ptr(), d_o.data_ptr(),
            dq.data_ptr(), dk.data_ptr(), dv.data_ptr())
    dims = (B, S_q, S_kv, D_qk, D_v, scale, p, int(causal), seed, off, h)
    if noalloc:
        rc = L.sdpa_hip_bwd_noalloc(dcode, *args, *dims)
    else:
        ws_bytes = int(L.sdpa_hip_bwd_workspace_bytes(B, S_q))
        ws = torch.empty((max(ws_bytes, 1),), dtype=torch.uint8, device=DEV)
        rc = L.sdpa_hip_bwd(dcode, *args, ws.data_ptr(), ws_bytes, *dims)
    assert rc == 0, pkg.status_string(rc)
    torch.cuda.synchronize()
    return dq, dk, dv


def test_noalloc_matches_workspace_entry(pkg):
    for case in CASES:  # in order: each call after the first is smaller than the first
        print(f"[case] noalloc {case}", flush=True)
        got = _run(pkg, case, True)
        ref = _run(pkg, case, False)
        for a, b in zip(got, ref):
            assert torch.equal(a, b)
            assert torch.isfinite(a.float()).all()


def test_noalloc_rejects_beyond_scratch(pkg):
    L = pkg.library()
    rows = (16 << 20) // 8  # 8 bytes per query row
    null = None
    call = lambda B, S: L.sdpa_hip_bwd_noalloc(1, null, null, null, null, null, null, null, null,
                                               null, B, S, S, 8, 8, 1.0, 0.0, 0, 0, 0, null)
    assert call(2, rows // 2 + 1) == pkg.SDPA_ERR_SCRATCH_LIMIT
    assert call(1, rows + 64) == pkg.SDPA_ERR_SCRATCH_LIMIT
