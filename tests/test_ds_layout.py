"""Layouts of the stored dS of the backward's dS path (DsLayoutT,
DsLayout::slot, DsLayout32::slot32 in csrc/sdpa_params.h), checked on the CPU:
tests/host/ds_layout.hip includes the header and checks, over a grid of
lengths with and without the causal mask, the closed-form chunk walk against
the dK/dV kernel's own walk, that chunks do not overlap and stay inside the
workspace, that every chunk the dQ kernels read was written, and inside a
chunk that both slot maps are one to one, that each store instruction of the
dK/dV kernels writes one whole KB, and that the fp32 dQ kernel's reads of a
key row fall in 32 different LDS banks.  The GPU side is covered by
tests/test_ds_path_gpu.py, which decodes the stored dS through the same maps."""
import os
import shutil
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(ROOT, "tf-custom-flash-attention_amd", "csrc")
HIPCC = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"


def test_ds_layouts(tmp_path):
    if not os.path.exists(HIPCC):
        pytest.skip("hipcc not found")
    exe = tmp_path / "ds_layout"
    subprocess.run([HIPCC, "-std=c++20", "-O1", "--offload-arch=gfx950", "-Xclang", "-target-feature", "-Xclang",
                    "-packed-fp32-ops", f"-I{os.path.join(ROOT, 'include')}", f"-I{CSRC}",
                    os.path.join(HERE, "host", "ds_layout.hip"), "-o", str(exe)],
                   check=True, capture_output=True)
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stdout + r.stderr
    assert r.stdout.startswith("ok")
