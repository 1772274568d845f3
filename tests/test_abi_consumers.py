"""Callers of the C ABIs written in C and C++ (tests/abi/): the public
headers compile with plain gcc / g++ (no HIP header, no platform macro),
and the entry points behave for them as for the ctypes binding.  The C and
C++ programs are compiled here, in the CPU suite, and run their own checks
(validation codes and messages, status strings, the host kernels on closed
forms).  The GPU caller, built by __graft_entry__.build(), allocates with
hipMalloc, launches on its own stream and is checked against the oracle."""
import os
import subprocess

import numpy as np
import pytest

from _common import TOL, Cfg, make_inputs, maxabs, oracle_kw

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
PKG = os.path.join(ROOT, "tf-custom-flash-attention_amd")
INC = os.path.join(ROOT, "include")


def _build_and_run(tmp_path, compiler, src, extra):
    exe = tmp_path / os.path.basename(src).replace(".", "_")
    cmd = [compiler, *extra, "-Wall", "-Wextra", "-Werror", f"-I{INC}", os.path.join(HERE, "abi", src),
           "-o", str(exe), f"-L{PKG}", "-lsdpa_hip", "-lsdpa_cpu", f"-Wl,-rpath,{PKG}"]
    if compiler == "gcc":
        cmd.append("-lm")
    subprocess.run(cmd, check=True)
    return subprocess.run([str(exe)], capture_output=True, text=True)


@pytest.mark.parametrize("compiler,src,extra", [("gcc", "consumer.c", ["-std=c11"]),
                                                ("g++", "consumer.cc", ["-std=c++17"])])
def test_abi_consumer_programs(pkg, tmp_path, compiler, src, extra):
    pkg.library()  # the libraries are built
    r = _build_and_run(tmp_path, compiler, src, extra)
    assert r.returncode == 0, r.stderr
    assert "ok" in r.stdout


@pytest.mark.gpu
@pytest.mark.parametrize("c", [
    Cfg("cxx_f16_causal", "f16", 2, 300, 300, 128, 128, True, 0.1, 128 ** -0.5, 7, 5),
    Cfg("cxx_f32_cross", "f32", 2, 70, 130, 64, 32, False, 0.2, 0.125, 42, 1000),
], ids=lambda c: c.name)
def test_gpu_caller_program(pkg, O, tmp_path, c):
    exe = os.path.join(HERE, "abi", "gpu_caller")
    assert os.path.exists(exe), "tests/abi/gpu_caller is not built: run __graft_entry__.build()"
    q, k, v, d_o = make_inputs(c)
    for name, a in (("q", q), ("k", k), ("v", v), ("do", d_o)):
        np.ascontiguousarray(a).tofile(tmp_path / f"{name}.bin")
    print(f"[case] gpu_caller {c.name}", flush=True)
    args = [exe, str(tmp_path), "1" if c.dtype == "f16" else "0", c.B, c.S_q, c.S_kv, c.D_qk, c.D_v,
            int(c.causal), repr(c.dropout), repr(c.scale), c.seed, c.offset]
    r = subprocess.run([str(a) for a in args], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stderr
    dt = np.float16 if c.dtype == "f16" else np.float32
    load = lambda n, shape, t=dt: np.fromfile(tmp_path / f"{n}.bin", dtype=t).reshape(shape)
    o = load("o", (c.B, c.S_q, c.D_v))
    s = load("stats", (c.B, c.S_q), np.float32)
    g = [load(n, a.shape) for n, a in (("dq", q), ("dk", k), ("dv", v))]
    tol = TOL[c.dtype]
    o_ref, s_ref = O.sdpa_fwd_gate(q, k, v, **oracle_kw(c))
    assert maxabs(o, o_ref) <= tol["o"] and maxabs(s, s_ref) <= tol["stats"]
    for a, ref in zip(g, O.sdpa_bwd_gate(q, k, v, o, s, d_o, **oracle_kw(c))):
        assert maxabs(a, ref) <= tol["grad"]
