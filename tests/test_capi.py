"""CPU tests of the C ABI (include/sdpa_hip.h): the library loads, exports
every declared symbol, and rejects bad arguments with the reference's
messages (sdpa/sdpa_cpu.cc:37-69,116-168; sdpa/sdpa_ops.cc:22-25,55-57)
before any device work.  No kernel is launched here."""
import ctypes
import os
import re
import subprocess

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "sdpa_hip.h")


def declared_symbols():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"\b(sdpa_hip_\w+)\s*\(", text)))


def test_every_declared_symbol_is_exported(pkg):
    L = pkg.library()
    syms = declared_symbols()
    assert len(syms) >= 9
    out = subprocess.run(["nm", "-D", "--defined-only", pkg.LIB_PATH], capture_output=True,
                         text=True, check=True).stdout
    exported = set(re.findall(r"\bT (\w+)$", out, re.M))
    for s in syms:
        assert s in exported, s
        assert hasattr(L, s)


def test_library_has_gfx950_code_object(pkg):
    # the offload bundle's target id names the architecture
    data = open(pkg.LIB_PATH, "rb").read()
    assert b"amdgcn-amd-amdhsa--gfx950" in data


REF_MESSAGES = {
    1: "seed must be scalar",
    2: "offset must be scalar",
    3: "K batch size mismatch",
    4: "K feature size mismatch",
    5: "V batch size mismatch",
    6: "V seq size mismatch",
    7: "O batch size mismatch",
    8: "O seq size mismatch",
    9: "O feature size mismatch",
    10: "dO batch size mismatch",
    11: "dO seq size mismatch",
    12: "dO feature size mismatch",
    13: "S batch size mismatch",
    14: "S seq size mismatch",
    15: "seq size Q != K while causal_mask = True",
    16: "CUDA kernel does not support feature size over 128. Set smaller feature size or use more heads",
}


def test_status_strings(pkg):
    for code, msg in REF_MESSAGES.items():
        assert pkg.status_string(code) == msg
    for code in range(0, 26):
        assert pkg.status_string(code) != "unknown sdpa status"


class Shape:
    """A stand-in with only a .shape, enough for the host-side checks."""

    def __init__(self, *dims):
        self.shape = dims


@pytest.fixture
def torch_shapes():
    torch = pytest.importorskip("torch")
    return lambda *d: torch.empty(d, device="meta")


FWD_CASES = [
    # q, k, v, seed, offset, causal, expected message
    ((2, 4, 8), (2, 4, 8), (2, 4, 8), (), (), False, None),
    ((2, 4, 8), (2, 4, 8), (2, 4, 8), (1,), (), False, "seed must be scalar"),
    ((2, 4, 8), (2, 4, 8), (2, 4, 8), (), (3,), False, "offset must be scalar"),
    ((2, 4, 8), (3, 4, 8), (2, 4, 8), (), (), False, "K batch size mismatch"),
    ((2, 4, 8), (2, 4, 9), (2, 4, 8), (), (), False, "K feature size mismatch"),
    ((2, 4, 8), (2, 4, 8), (3, 4, 8), (), (), False, "V batch size mismatch"),
    ((2, 4, 8), (2, 4, 8), (2, 5, 8), (), (), False, "V seq size mismatch"),
    ((2, 4, 8), (2, 6, 8), (2, 6, 8), (), (), True, "seq size Q != K while causal_mask = True"),
    ((2, 4, 129), (2, 4, 129), (2, 4, 8), (), (), False, "CUDA kernel does not support feature size"),
    ((2, 4, 8), (2, 4, 8), (2, 4, 200), (), (), False, "CUDA kernel does not support feature size"),
    ((4, 8), (2, 4, 8), (2, 4, 8), (), (), False, "Shape must be rank 3"),
]


@pytest.mark.parametrize("case", FWD_CASES)
def test_forward_validation(pkg, torch_shapes, case):
    qs, ks, vs, seed, off, causal, msg = case
    seed_t = torch_shapes(*seed) if seed else 0
    off_t = torch_shapes(*off) if off else 0
    args = (torch_shapes(*qs), torch_shapes(*ks), torch_shapes(*vs), seed_t, off_t, causal)
    if msg is None:
        pkg.check_fwd(*args)
    else:
        with pytest.raises(pkg.InvalidArgumentError, match=re.escape(msg)):
            pkg.check_fwd(*args)


BWD_OK = dict(q=(2, 4, 8), k=(2, 6, 8), v=(2, 6, 5), o=(2, 4, 5), s=(2, 4), do=(2, 4, 5))
BWD_CASES = [
    ({}, False, None),
    (dict(o=(3, 4, 5)), False, "O batch size mismatch"),
    (dict(o=(2, 5, 5)), False, "O seq size mismatch"),
    (dict(o=(2, 4, 6)), False, "O feature size mismatch"),
    (dict(do=(1, 4, 5)), False, "dO batch size mismatch"),
    (dict(do=(2, 3, 5)), False, "dO seq size mismatch"),
    (dict(do=(2, 4, 4)), False, "dO feature size mismatch"),
    (dict(s=(1, 4)), False, "S batch size mismatch"),
    (dict(s=(2, 7)), False, "S seq size mismatch"),
    ({}, True, "seq size Q != K while causal_mask = True"),
    (dict(k=(2, 6, 7)), False, "K feature size mismatch"),
    (dict(v=(2, 7, 5)), False, "V seq size mismatch"),
]


@pytest.mark.parametrize("case", BWD_CASES)
def test_backward_validation(pkg, torch_shapes, case):
    over, causal, msg = case
    sh = {**BWD_OK, **over}
    args = [torch_shapes(*sh[n]) for n in ("q", "k", "v", "o", "s", "do")]
    if msg is None:
        pkg.check_bwd(*args, 0, 0, causal)
    else:
        with pytest.raises(pkg.InvalidArgumentError, match=re.escape(msg)):
            pkg.check_bwd(*args, 0, 0, causal)


def test_launch_entry_points_reject_before_device_work(pkg):
    """Argument errors return before any HIP call (null pointers are never
    touched), so these run without a GPU."""
    L = pkg.library()
    null = None
    fwd = lambda dtype, B, S_q, S_kv, D_qk, D_v, p, causal: L.sdpa_hip_fwd(
        dtype, null, null, null, null, null, B, S_q, S_kv, D_qk, D_v, 1.0, p, causal, 0, 0, null)
    assert fwd(2, 1, 4, 4, 8, 8, 0.0, 0) == 18          # SDPA_ERR_DTYPE
    assert fwd(1, -1, 4, 4, 8, 8, 0.0, 0) == 19         # negative dim
    assert fwd(1, 1, 4, 5, 8, 8, 0.0, 1) == 15          # causal with S_q != S_kv
    assert fwd(1, 1, 4, 4, 8, 129, 0.0, 0) == 16        # feature size over 128
    assert fwd(1, 1, 4, 4, 8, 8, 1.0, 0) == 21          # dropout == 1
    assert fwd(1, 1, 4, 4, 8, 8, 1.5, 0) == 20          # dropout > 1 passes the checks (drops all)
    assert fwd(1, 0, 4, 4, 8, 8, 0.0, 0) == 0           # empty: nothing to do
    assert fwd(1, 1, 4, 4, 8, 8, 0.0, 0) == 20          # null pointers for non-empty tensors
    bwd = lambda ws_bytes: L.sdpa_hip_bwd(1, null, null, null, null, null, null, null, null, null,
                                          null, ws_bytes, 2, 4, 4, 8, 8, 1.0, 0.0, 0, 0, 0, null)
    assert bwd(0) == 22                                  # workspace too small
    assert L.sdpa_hip_bwd_workspace_bytes(2, 4) == 256
    # two fp32 rows per query row: stats * log2(e) and delta
    assert L.sdpa_hip_bwd_workspace_bytes(128, 4096) == 2 * 128 * 4096 * 4
    assert L.sdpa_hip_bwd_workspace_bytes(0, 4096) == 0


def _ds_chunks(S_q, S_kv, causal, qbk=64):
    """Query blocks (qbk rows: 64 in the fp16 split dK/dV kernel, 32 in the
    fp32 one) the kernel visits, summed over its key tiles (128 keys): the dS
    chunks of one batch row, counted the way the kernels walk them (q_begin
    and the block count of sdpa_f16_dkdv_split.hip and of
    sdpa_bwd_dkdv_f32_split_kernel)."""
    n = 0
    for kt in range((S_kv + 127) // 128):
        q_begin = (min(128 * kt, S_q) // qbk) * qbk if causal else 0
        n += (S_q - q_begin + qbk - 1) // qbk
    return n


def test_ds_workspace_bytes(pkg):
    """sdpa_hip_bwd_workspace_bytes_ds = the per-row workspace + 16 KB per
    visited (key tile, query block) per batch row, for float16 (query blocks
    of 64) and float32 (blocks of 32) with a feature size over 64; the
    per-row size for every other shape."""
    L = pkg.library()
    for B, S_q, S_kv, D_qk, D_v, causal in [(128, 4096, 4096, 128, 128, 1), (3, 333, 333, 128, 128, 1),
                                             (2, 130, 300, 128, 64, 0), (2, 300, 100, 64, 128, 0),
                                             (1, 1, 1, 128, 128, 1), (1, 31, 1000, 80, 80, 0),
                                             (5, 1000, 1000, 96, 96, 1), (2, 64, 64, 128, 128, 1)]:
        rows = L.sdpa_hip_bwd_workspace_bytes(B, S_q)
        want = rows + B * _ds_chunks(S_q, S_kv, causal) * 16384
        assert L.sdpa_hip_bwd_workspace_bytes_ds(1, B, S_q, S_kv, D_qk, D_v, causal) == want
        want32 = rows + B * _ds_chunks(S_q, S_kv, causal, 32) * 16384
        assert L.sdpa_hip_bwd_workspace_bytes_ds(0, B, S_q, S_kv, D_qk, D_v, causal) == want32
        # both sides <= 64: the per-row workspace only
        assert L.sdpa_hip_bwd_workspace_bytes_ds(1, B, S_q, S_kv, 64, 64, causal) == rows
        assert L.sdpa_hip_bwd_workspace_bytes_ds(0, B, S_q, S_kv, 64, 64, causal) == rows
    # c4: 1056 chunks per batch row under the causal mask (half of 32 x 64, plus the diagonal)
    assert _ds_chunks(4096, 4096, True) == 1056
    # c5 in fp32: 128 key tiles x 16 query blocks per batch row (2 GiB at B = 64)
    assert _ds_chunks(512, 16384, False, 32) == 2048
    assert L.sdpa_hip_bwd_workspace_bytes_ds(1, 0, 4096, 4096, 128, 128, 1) == 0
    assert L.sdpa_hip_bwd_workspace_bytes_ds(1, 2, 64, 0, 128, 128, 0) == L.sdpa_hip_bwd_workspace_bytes(2, 64)


def test_ds_phase_rejects_before_device_work(pkg):
    """sdpa_hip_bwd_ds_phase returns SDPA_ERR_DS_PATH where sdpa_hip_bwd would
    not take the dS path; the stand-in addresses (16-byte aligned, never
    dereferenced on the host) are refused before any launch."""
    L = pkg.library()
    fake = 4096
    big = 1 << 40

    def phase(ph, dtype, D_qk=128, D_v=128, ws=big, B=2):
        return L.sdpa_hip_bwd_ds_phase(ph, dtype, *([fake] * 10), ws, B, 64, 64, D_qk, D_v, 1.0, 0.0, 1, 0, 0,
                                       None)
    assert phase(1, 1, 64, 64) == pkg.SDPA_ERR_DS_PATH         # both sides <= 64
    assert phase(0, 0, 64, 64) == pkg.SDPA_ERR_DS_PATH         # fp32, both sides <= 64
    small32 = L.sdpa_hip_bwd_workspace_bytes_ds(0, 2, 64, 64, 128, 128, 1) - 1
    assert phase(1, 0, ws=small32) == pkg.SDPA_ERR_DS_PATH     # fp32 workspace one byte short
    assert phase(3, 1) == pkg.SDPA_ERR_DS_PATH                 # no such phase
    assert phase(-1, 1) == pkg.SDPA_ERR_DS_PATH
    small = L.sdpa_hip_bwd_workspace_bytes_ds(1, 2, 64, 64, 128, 128, 1) - 1
    assert phase(2, 1, ws=small) == pkg.SDPA_ERR_DS_PATH       # workspace one byte short
    assert phase(2, 1, ws=0) == 22                             # below even the per-row workspace
    assert phase(0, 1, B=0) == 0                               # empty: nothing to do


def test_drop_threshold_values(pkg):
    assert pkg.drop_threshold(0.1) == 0x19999991
    assert pkg.drop_threshold(0.2) == 0x33333321
    assert pkg.drop_threshold(0.0) == 0
    assert pkg.drop_threshold(-0.5) == 0
    assert pkg.drop_threshold(float("nan")) == 0
    assert pkg.drop_threshold(1.5) == 1 << 32


def test_python_wrapper_rejects_cpu_tensors(pkg):
    torch = pytest.importorskip("torch")
    q = torch.zeros((1, 4, 8), dtype=torch.float16)
    with pytest.raises(pkg.InvalidArgumentError):
        pkg.sdpa(q, q, q, 0, 0)
