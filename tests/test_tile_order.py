"""Work order of the fp16 DMA kernels (xcd_map and row_window in
csrc/sdpa_dma.h), checked on the CPU: tests/host/tile_order.hip includes the
header, runs xcd_map on the host over a grid of batch sizes (multiples of 8
and not), tile counts and chunk caps, and checks that workgroup ids map one
to one onto (batch, tile), that each XCD covers its contiguous range of the
batch-major tile list, that it runs that range as the fewest equal chunks of
at most wcap rows' worth of tiles, each rank-major (heaviest tiles of all its
rows first), that chunks are whole rows where wcap divides B / 8, and the
row_window rule.  The GPU side of the same mapping is covered by the
all-batch parity checks of c3/c4 (B = 256 and 128) and the B = 12, 16, 24
and 36 edge shapes."""
import os
import shutil
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(ROOT, "tf-custom-flash-attention_amd", "csrc")
HIPCC = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"


def test_work_order(tmp_path):
    if not os.path.exists(HIPCC):
        pytest.skip("hipcc not found")
    exe = tmp_path / "tile_order"
    subprocess.run([HIPCC, "-std=c++20", "-O1", "--offload-arch=gfx950", "-Xclang", "-target-feature", "-Xclang",
                    "-packed-fp32-ops", f"-I{os.path.join(ROOT, 'include')}", f"-I{CSRC}",
                    os.path.join(HERE, "host", "tile_order.hip"), "-o", str(exe)],
                   check=True, capture_output=True)
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stdout + r.stderr
    assert r.stdout.startswith("ok")
