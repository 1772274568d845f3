"""The host (CPU) kernels of the op's DEVICE_CPU registration
(libsdpa_cpu.so, include/sdpa_cpu.h) against the CPU oracle with the
reference CPU functors' gates (dropout iff p > 0, skip P < 1e-6;
sdpa/sdpa_cpu.cc:232-235,384-385), at the north_star tolerances: fp32 within
1e-5, fp16 within 2e-3 on o and 1e-2 on the gradients; dropout masks bit-exact
(read back through the kernels with selector inputs, as the GPU tests do)."""
import numpy as np
import pytest

from _common import CONFIGS, TOL, Cfg, argmax_grad, make_inputs, maxabs

# CPU-sized cases: c1 and c2 as configured, then shapes that cover the tile
# tails (16 query rows, 64 keys), the causal mask, D_qk != D_v and dropout.
CASES = [CONFIGS[0], CONFIGS[1],
         Cfg("causal_f16_p01", "f16", 3, 150, 150, 64, 64, True, 0.1, 0.125, 7, 3),
         Cfg("causal_f32_p02", "f32", 2, 97, 97, 128, 32, True, 0.2, 128 ** -0.5, 11, 2**40),
         Cfg("cross_f16", "f16", 2, 33, 257, 100, 36, False, 0.05, 0.1, 5, 6),
         Cfg("tiny_f32", "f32", 2, 1, 1, 8, 8, False, 0.0, 1.0),
         Cfg("d1_f16", "f16", 1, 50, 50, 1, 1, True, 0.0, 1.0)]


@pytest.fixture(scope="module")
def host(pkg):
    import importlib
    return importlib.import_module(pkg.__name__ + ".host")


@pytest.mark.parametrize("c", CASES, ids=[c.name for c in CASES])
def test_host_kernels_match_oracle(host, O, c):
    q, k, v, d_o = make_inputs(c)
    kw = dict(scale=c.scale, dropout=c.dropout, causal_mask=c.causal, seed=c.seed, offset=c.offset)
    o, s = host.sdpa(q, k, v, **kw)
    o_ref, s_ref = O.sdpa_fwd_gate(q, k, v, gpu_gates=False, **kw)
    if c.do_kind == "argmax":
        d_o = argmax_grad(o_ref)
    tol = TOL[c.dtype]
    assert maxabs(o, o_ref) <= tol["o"]
    assert maxabs(s, s_ref) <= tol["stats"]
    g = host.sdpa_grad(q, k, v, o, s, d_o, **kw)
    g_ref = O.sdpa_bwd_gate(q, k, v, o, s, d_o, gpu_gates=False, **kw)
    for name, a, r in zip(("dq", "dk", "dv"), g, g_ref):
        assert maxabs(a, r) <= tol["grad"], name


@pytest.mark.parametrize("causal", [False, True])
def test_host_kernels_dropout_mask_bit_exact(host, O, causal):
    """Selector inputs expose single elements (q = 0 makes P uniform):
    forward o[i, d] > 0 iff (i, d) kept, with one-hot V; dV[j, d] > 0 iff
    (d, j) kept, with one-hot dO.  Compared bit for bit with the reference
    predicate u < p."""
    B, S, D, p, seed, off = 2, 40, 40, 0.3, 42, 1000
    ref = O.keep_mask(B, S, S, p, seed, off)
    if causal:
        ref &= np.tril(np.ones((S, S), np.uint8))[None]
    q = np.zeros((B, S, D), np.float32)
    k = np.random.default_rng(0).standard_normal((B, S, D)).astype(np.float32)
    eye = np.broadcast_to(np.eye(S, D, dtype=np.float32), (B, S, D)).copy()
    kw = dict(scale=1.0, dropout=p, causal_mask=causal, seed=seed, offset=off)
    o, s = host.sdpa(q, k, eye, **kw)
    assert np.array_equal((o > 0).astype(np.uint8), ref)
    _, _, dv = host.sdpa_grad(q, k, eye, o, s, eye, **kw)
    assert np.array_equal((dv > 0).astype(np.uint8).transpose(0, 2, 1), ref)


def test_host_kernels_edge_cases(host, pkg):
    z = lambda *s: np.zeros(s, np.float32)
    # no keys: o = 0 and stats = -1e9 + log(1e-6) (sdpa_cpu.cc:302-308)
    o, s = host.sdpa(z(2, 3, 8), z(2, 0, 8), z(2, 0, 4))
    assert np.all(o == 0)
    assert np.all(s == np.float32(-1e9) + np.float32(np.log(np.float32(1e-6))))
    # empty batch: nothing to do
    o, s = host.sdpa(z(0, 3, 8), z(0, 3, 8), z(0, 3, 4))
    assert o.shape == (0, 3, 4)
    # argument errors carry the reference's messages
    with pytest.raises(pkg.InvalidArgumentError, match="seq size Q != K while causal_mask = True"):
        host.sdpa(z(1, 3, 8), z(1, 4, 8), z(1, 4, 8), causal_mask=True)
    with pytest.raises(pkg.InvalidArgumentError, match="feature size over 128"):
        host.sdpa(z(1, 3, 130), z(1, 3, 130), z(1, 3, 8))


def test_host_kernels_thread_count_invariant(host):
    """Work items own disjoint outputs: the result does not depend on the
    number of threads."""
    c = Cfg("threads", "f16", 3, 70, 70, 32, 32, True, 0.2, 0.2, 1, 2)
    q, k, v, d_o = make_inputs(c)
    kw = dict(scale=c.scale, dropout=c.dropout, causal_mask=True, seed=1, offset=2)
    outs = []
    for nt in (1, 3, 8):
        o, s = host.sdpa(q, k, v, nthreads=nt, **kw)
        outs.append([o, s, *host.sdpa_grad(q, k, v, o, s, d_o, nthreads=nt, **kw)])
    for other in outs[1:]:
        for a, b in zip(outs[0], other):
            assert np.array_equal(a, b)


@pytest.mark.parametrize("dtype", ["f32", "f16"])
def test_host_kernels_dropout_above_one(host, O, pkg, dtype):
    """dropout > 1 drops every element, as in the reference (u <= 1 < p): o = 0,
    the usual statistics, dV = 0 and dS = -P delta for every element (the
    backward is run on an o that is not 0, so delta != 0).  dropout == 1 is
    rejected (the reference would scale the rare u == 1 elements by 1 / 0)."""
    c = Cfg("above_one", dtype, 2, 70, 70, 48, 24, True, 1.5, 0.2, 3, 5)
    q, k, v, d_o = make_inputs(c)
    kw = dict(scale=c.scale, dropout=c.dropout, causal_mask=c.causal, seed=c.seed, offset=c.offset)
    o, s = host.sdpa(q, k, v, **kw)
    o_ref, s_ref = O.sdpa_fwd_gate(q, k, v, gpu_gates=False, **kw)
    assert np.all(o == 0) and np.all(o_ref == 0)
    assert maxabs(s, s_ref) <= TOL[dtype]["stats"]
    o_in, _ = host.sdpa(q, k, v, **dict(kw, dropout=0.0))
    g = host.sdpa_grad(q, k, v, o_in, s, d_o, **kw)
    g_ref = O.sdpa_bwd_gate(q, k, v, o_in, s, d_o, gpu_gates=False, **kw)
    assert np.all(g[2] == 0)
    for name, a, r in zip(("dq", "dk", "dv"), g, g_ref):
        assert maxabs(a, r) <= TOL[dtype]["grad"], name
    assert np.abs(g_ref[0].astype(np.float32)).max() > 1e-2
    with pytest.raises(pkg.InvalidArgumentError, match="dropout must not be 1"):
        host.sdpa(q, k, v, **dict(kw, dropout=1.0))


def test_host_binding_checks_before_reading(host, pkg, monkeypatch):
    """The numpy binding runs the op's checks (sdpa/sdpa_cpu.cc:37-69,
    116-168) and the dtype rules before any data is read, through
    libsdpa_cpu.so alone: the GPU library is made unloadable here."""
    monkeypatch.setattr(pkg, "LIB_PATH", "/nonexistent/libsdpa_hip.so")
    monkeypatch.setattr(pkg, "_lib", None)
    f = lambda *s, dt=np.float32: np.zeros(s, dt)
    E = pkg.InvalidArgumentError
    with pytest.raises(E, match="K batch size mismatch"):      # q [4,16,8] against k, v [1,16,8]
        host.sdpa(f(4, 16, 8), f(1, 16, 8), f(1, 16, 8))
    with pytest.raises(E, match="K feature size mismatch"):
        host.sdpa(f(2, 16, 8), f(2, 16, 6), f(2, 16, 8))
    with pytest.raises(E, match="V seq size mismatch"):
        host.sdpa(f(2, 16, 8), f(2, 16, 8), f(2, 15, 8))
    with pytest.raises(E, match="rank 3"):
        host.sdpa(f(16, 8), f(16, 8), f(16, 8))
    with pytest.raises(E, match="seed must be scalar"):
        host.sdpa(f(2, 4, 8), f(2, 4, 8), f(2, 4, 8), seed=np.array([1, 2]))
    with pytest.raises(E, match="k has dtype float16"):
        host.sdpa(f(2, 4, 8), f(2, 4, 8, dt=np.float16), f(2, 4, 8))
    with pytest.raises(E, match="T must be half or float"):
        host.sdpa(f(2, 4, 8, dt=np.float64), f(2, 4, 8, dt=np.float64), f(2, 4, 8, dt=np.float64))
    q, kv, o, s = f(2, 4, 8), f(2, 6, 8), f(2, 4, 8), f(2, 4)
    with pytest.raises(E, match="O seq size mismatch"):
        host.sdpa_grad(q, kv, kv, f(2, 5, 8), s, o)
    with pytest.raises(E, match="dO feature size mismatch"):
        host.sdpa_grad(q, kv, kv, o, s, f(2, 4, 7))
    with pytest.raises(E, match="S batch size mismatch"):
        host.sdpa_grad(q, kv, kv, o, f(3, 4), o)
    with pytest.raises(E, match="stats must be float32"):
        host.sdpa_grad(q, kv, kv, o, s.astype(np.float16), o)
    with pytest.raises(E, match="d_o has dtype float16"):
        host.sdpa_grad(q, kv, kv, o, s, o.astype(np.float16))
    with pytest.raises(E, match="dropout must not be 1"):        # a kernel-side check, same messages
        host.sdpa(f(2, 4, 8), f(2, 4, 8), f(2, 4, 8), dropout=1.0)
    assert pkg._lib is None  # the GPU library was never loaded
