"""The TensorFlow-ROCm op layer (tf-custom-flash-attention_amd/tf_op/).

* Without TensorFlow: the op definitions in sdpa_ops.cc declare the
  reference's interface exactly (sdpa/sdpa_ops.cc:7-63: op names, input /
  output names, types and order, attribute names, defaults and order), and
  sdpa_kernels.cc registers both ops for DEVICE_CPU and DEVICE_GPU x
  {float, half} with seed / offset in host memory on the GPU
  (sdpa/sdpa_cpu.cc:460-488).
* Without TensorFlow: sdpa.py runs against a stand-in tensorflow module that
  records the library it loads, the forward call and the gradient's SdpaGrad
  call (inputs, attributes, return arity), as the reference wires them
  (test.py:12-30); planted wiring mistakes fail that check.
* With TensorFlow: build.sh builds sdpa_rocm.so, sdpa.py loads it, and the
  op plus its registered gradient agree with the oracle on the CPU and, on a
  GPU, with the oracle at the north_star tolerances.  TensorFlow is not
  installed in this image nor on the GPU boxes, so these skip with that
  reason.
"""
import importlib.util
import os
import re
import subprocess

import numpy as np
import pytest

from _common import TOL, Cfg, make_inputs, maxabs, oracle_kw

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
TF_OP = os.path.join(ROOT, "tf-custom-flash-attention_amd", "tf_op")

# The reference's op interface (sdpa/sdpa_ops.cc:7-63), in declaration order.
REFERENCE_OPS = {
    "Sdpa": {
        "Input": ["q: T", "k: T", "v: T", "seed: uint64", "offset: uint64"],
        "Attr": ["scale: float = 1.0", "dropout: float = 0.0", "causal_mask: bool = false",
                 "T: {half, float}"],
        "Output": ["output: T", "stats: float"],
    },
    "SdpaGrad": {
        "Input": ["q: T", "k: T", "v: T", "out: T", "stats: float", "do: T", "seed: uint64",
                  "offset: uint64"],
        "Attr": ["dropout: float = 0.0", "scale: float = 1.0", "causal_mask: bool = false",
                 "T: {half, float}"],
        "Output": ["dq: T", "dk: T", "dv: T"],
    },
}


def _registered_ops(text):
    ops = {}
    for m in re.finditer(r'REGISTER_OP\("(\w+)"\)(.*?);', text, re.S):
        chain = re.sub(r"//[^\n]*", "", m.group(2))
        entry = {"Input": [], "Attr": [], "Output": []}
        for kind, spec in re.findall(r'\.(Input|Attr|Output)\("([^"]*)"\)', chain):
            entry[kind].append(spec)
        entry["shape_fn"] = ".SetShapeFn(" in chain
        ops[m.group(1)] = entry
    return ops


def test_op_definitions_match_reference_interface():
    ops = _registered_ops(open(os.path.join(TF_OP, "sdpa_ops.cc")).read())
    assert set(ops) == set(REFERENCE_OPS)
    for name, want in REFERENCE_OPS.items():
        for kind in ("Input", "Attr", "Output"):
            assert ops[name][kind] == want[kind], (name, kind)
        assert ops[name]["shape_fn"]


def test_kernel_registrations():
    text = open(os.path.join(TF_OP, "sdpa_kernels.cc")).read()
    cpu = re.search(r"#define SDPA_REGISTER_CPU\(T\)(.*?)#undef SDPA_REGISTER_CPU", text, re.S).group(1)
    gpu = re.search(r"#define SDPA_REGISTER_GPU\(T\)(.*?)#undef SDPA_REGISTER_GPU", text, re.S).group(1)
    for block, dev in ((cpu, "DEVICE_CPU"), (gpu, "DEVICE_GPU")):
        for op in ("Sdpa", "SdpaGrad"):
            assert re.search(rf'Name\("{op}"\)\.Device\({dev}\)\.TypeConstraint<T>\("T"\)', block), (op, dev)
        for t in ("float", "Eigen::half"):
            assert re.search(rf"SDPA_REGISTER_{dev[7:]}\({re.escape(t)}\);", text), (dev, t)
    assert gpu.count('.HostMemory("seed").HostMemory("offset")') == 2
    assert "HostMemory" not in cpu
    # the GPU path calls the HIP C ABI, the CPU path the host kernels
    assert "sdpa_hip_fwd(" in text and "sdpa_hip_bwd(" in text
    assert "sdpa_cpu_fwd(" in text and "sdpa_cpu_bwd(" in text


@pytest.fixture(scope="module")
def tf_sdpa():
    tf = pytest.importorskip(
        "tensorflow",
        reason="TensorFlow(-ROCm) is not installed in this image or on the GPU boxes: "
               "tf_op/build.sh cannot build sdpa_rocm.so and the op cannot be loaded here")
    lib = os.path.join(TF_OP, "sdpa_rocm.so")
    if not os.path.exists(lib):
        subprocess.run([os.path.join(TF_OP, "build.sh")], check=True)
    spec = importlib.util.spec_from_file_location("tf_op_sdpa", os.path.join(TF_OP, "sdpa.py"))
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return tf, mod


def _run_op(tf, mod, c, device):
    q, k, v, d_o = make_inputs(c)
    with tf.device(device):
        tq, tk, tv = (tf.constant(a) for a in (q, k, v))
        seed = tf.constant(c.seed, dtype=tf.uint64)
        off = tf.constant(c.offset, dtype=tf.uint64)
        with tf.GradientTape() as tape:
            tape.watch([tq, tk, tv])
            o, s = mod.sdpa(tq, tk, tv, seed, off, dropout=c.dropout, scale=c.scale,
                            causal_mask=c.causal)
        grads = tape.gradient(o, [tq, tk, tv], output_gradients=tf.constant(d_o))
    return (q, k, v, d_o), o.numpy(), s.numpy(), [g.numpy() for g in grads]


CASES = [Cfg("tf_f32", "f32", 2, 64, 64, 32, 16, True, 0.1, 32 ** -0.5, 42, 1000),
         Cfg("tf_f16", "f16", 2, 96, 96, 64, 64, False, 0.2, 0.125, 7, 0)]


@pytest.mark.parametrize("c", CASES, ids=lambda c: c.name)
def test_tf_op_cpu(tf_sdpa, O, c):
    tf, mod = tf_sdpa
    (q, k, v, d_o), o, s, grads = _run_op(tf, mod, c, "/CPU:0")
    kw = dict(oracle_kw(c), gpu_gates=False)
    o_ref, s_ref = O.sdpa_fwd_gate(q, k, v, **kw)
    assert maxabs(o, o_ref) <= TOL[c.dtype]["o"]
    for g, r in zip(grads, O.sdpa_bwd_gate(q, k, v, o, s, d_o, **kw)):
        assert maxabs(g, r) <= TOL[c.dtype]["grad"]


@pytest.mark.gpu
@pytest.mark.parametrize("c", CASES, ids=lambda c: c.name)
def test_tf_op_gpu(tf_sdpa, O, c):
    tf, mod = tf_sdpa
    (q, k, v, d_o), o, s, grads = _run_op(tf, mod, c, "/GPU:0")
    o_ref, s_ref = O.sdpa_fwd_gate(q, k, v, **oracle_kw(c))
    assert maxabs(o, o_ref) <= TOL[c.dtype]["o"]
    for g, r in zip(grads, O.sdpa_bwd_gate(q, k, v, o, s, d_o, **oracle_kw(c))):
        assert maxabs(g, r) <= TOL[c.dtype]["grad"]


# ---- sdpa.py executed against a stand-in TensorFlow module -------------------
# TensorFlow is absent here, so the module's wiring is checked by running it
# against a recorder: the library it loads, the forward call, and the
# registered gradient's call of SdpaGrad (inputs, attributes, return arity),
# as the reference wires them (test.py:12-30, README.md:28-56).

class _Recorder:
    """The loaded op library: records every call, returns sentinels."""

    def __init__(self):
        self.calls = []

    def sdpa(self, *args, **kwargs):
        self.calls.append(("sdpa", args, kwargs))
        return ("o", "stats")

    def sdpa_grad(self, *args, **kwargs):
        self.calls.append(("sdpa_grad", args, kwargs))
        return ("dq", "dk", "dv")


def _fake_tensorflow():
    import types
    tf = types.ModuleType("tensorflow")
    tf.Tensor, tf.Operation = object, object
    tf.loaded, tf.gradients, tf.lib = [], {}, _Recorder()

    def load_op_library(path):
        tf.loaded.append(path)
        return tf.lib

    def RegisterGradient(name):
        def deco(fn):
            tf.gradients[name] = fn
            return fn
        return deco

    tf.load_op_library, tf.RegisterGradient = load_op_library, RegisterGradient
    return tf


class _FakeOp:
    """An Sdpa op as the gradient function sees it."""

    def __init__(self, inputs, outputs, attrs):
        self.inputs, self.outputs, self._attrs = inputs, outputs, attrs

    def get_attr(self, name):
        return self._attrs[name]


def _check_sdpa_module(path, monkeypatch):
    """Run the module at `path` against the stand-in and assert the
    reference's wiring; AssertionError on any difference."""
    tf = _fake_tensorflow()
    monkeypatch.setitem(__import__("sys").modules, "tensorflow", tf)
    monkeypatch.delenv("SDPA_ROCM_LIB", raising=False)
    spec = importlib.util.spec_from_file_location("sdpa_tf_module_under_test", path)
    m = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(m)
    assert tf.loaded == [os.path.join(os.path.dirname(path), "sdpa_rocm.so")]
    # forward: the op's positional inputs and keyword attributes, its outputs returned
    q, k, v, seed, offset = (object() for _ in range(5))
    assert m.sdpa(q, k, v, seed, offset, dropout=0.25, scale=0.125, causal_mask=True) == ("o", "stats")
    assert tf.lib.calls[-1] == ("sdpa", (q, k, v, seed, offset),
                                dict(dropout=0.25, scale=0.125, causal_mask=True))
    # the gradient registered for "Sdpa": SdpaGrad(q, k, v, o, stats, d_o, seed, offset)
    assert set(tf.gradients) == {"Sdpa"}
    o, stats, d_o, d_stats = (object() for _ in range(4))
    attrs = dict(dropout=0.3, scale=0.5, causal_mask=True)
    op = _FakeOp((q, k, v, seed, offset), (o, stats), attrs)
    grads = tf.gradients["Sdpa"](op, d_o, d_stats)
    assert tuple(grads) == ("dq", "dk", "dv", None, None)
    assert tf.lib.calls[-1] == ("sdpa_grad", (q, k, v, o, stats, d_o, seed, offset), attrs)
    # the library path can be overridden
    monkeypatch.setenv("SDPA_ROCM_LIB", "/elsewhere/sdpa_rocm.so")
    tf.loaded.clear()
    spec.loader.exec_module(importlib.util.module_from_spec(spec))
    assert tf.loaded == ["/elsewhere/sdpa_rocm.so"]


def test_sdpa_module_wiring_with_stand_in_tensorflow(monkeypatch):
    _check_sdpa_module(os.path.join(TF_OP, "sdpa.py"), monkeypatch)


@pytest.mark.parametrize("old,new", [
    ("o, stats = op.outputs", "stats, o = op.outputs"),                        # o and stats swapped
    ("d_o, seed, offset,", "d_o, offset, seed,"),                              # seed and offset swapped
    ("causal_mask=op.get_attr(\"causal_mask\"))", "causal_mask=False)"),       # attribute dropped
    ("return dq, dk, dv, None, None", "return dq, dk, dv, None"),              # wrong arity
    ("dropout=op.get_attr(\"dropout\"), scale=op.get_attr(\"scale\")",
     "dropout=op.get_attr(\"scale\"), scale=op.get_attr(\"dropout\")"),       # attributes crossed
    ("return mod.sdpa(q, k, v, seed, offset,", "return mod.sdpa(q, k, v, offset, seed,"),
])
def test_sdpa_module_check_catches_planted_mistakes(tmp_path, monkeypatch, old, new):
    src = open(os.path.join(TF_OP, "sdpa.py")).read()
    assert old in src
    planted = tmp_path / "sdpa.py"
    planted.write_text(src.replace(old, new))
    with pytest.raises(AssertionError):
        _check_sdpa_module(str(planted), monkeypatch)
