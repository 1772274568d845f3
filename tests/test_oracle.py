"""Pins the CPU oracle (oracle/sdpa_oracle.cc, restating sdpa/sdpa_cpu.cc)
before it is trusted as the parity checker of the HIP kernels.

* dropout hash: known answers of the counter's closed form
  ((seed + offset + (b S_q + i) S_kv + j) A + C mod 2^64, high word), the
  golden JSON written by an independent Python restatement, the linearity
  of the counter, and an exhaustive check over all 2^32 hash words that the reference's float
  predicate u < p equals the integer threshold used by the kernels;
* attention math: float64 dense attention fixtures (tests/golden), finite
  differences of the dense forward (pinning the closed-form gradients those
  fixtures hold), closed-form invariants;
* planted mistakes in copies of the checkers (wrong threshold, transposed
  operand, missing dropout rescale) must fail the same checks.
"""
import json
import os

import numpy as np
import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
GOLD = os.path.join(HERE, "golden")


def golden_dense():
    import importlib.util
    spec = importlib.util.spec_from_file_location("make_golden", os.path.join(GOLD, "make_golden.py"))
    m = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(m)
    return m


# ---------------------------------------------------------------------------
# dropout hash
# ---------------------------------------------------------------------------
KNOWN_ANSWERS = [
    ((42, 1000, 0, 0, 0, 400, 400), 0x91995BE0),
    ((42, 1000, 0, 0, 1, 400, 400), 0xE9EB500D),
    ((42, 1000, 0, 1, 0, 400, 400), 0x91A6E2A8),
    ((42, 1000, 19, 399, 399, 400, 400), 0xDFFB4727),
    ((7, 0, 0, 0, 0, 4096, 4096), 0x7E4328BC),
    ((7, 0, 127, 4095, 4095, 4096, 4096), 0xCC3BF425),
    ((7, 0, 5, 1000, 17, 4096, 4096), 0x5B427DB9),
]


@pytest.mark.parametrize("args,want", KNOWN_ANSWERS)
def test_rng_known_answers(O, args, want):
    assert O.rng_bits(*args) == want


def test_rng_matches_golden(O):
    with open(os.path.join(GOLD, "rng_known_answers.json")) as f:
        answers = json.load(f)
    assert len(answers) >= 10
    for a in answers:
        args = (a["seed"], a["offset"], a["b"], a["i"], a["j"], a["S_q"], a["S_kv"])
        assert O.rng_bits(*args) == a["bits"]
        assert O.rng_uniform(*args) == np.float32(a["u"])
        for p, dropped in a["dropped"].items():
            assert (O.rng_uniform(*args) < np.float32(float(p))) == dropped


def test_rng_counter_structure(O):
    # seed and offset only enter through their sum; the counter is linear in (b, i, j)
    assert O.rng_bits(42, 1000, 3, 5, 7, 400, 400) == O.rng_bits(1042, 0, 3, 5, 7, 400, 400)
    assert O.rng_bits(1, 2, 1, 0, 0, 9, 11) == O.rng_bits(1, 2, 0, 9, 0, 9, 11)
    assert O.rng_bits(1, 2, 0, 1, 0, 9, 11) == O.rng_bits(1, 2 + 11, 0, 0, 0, 9, 11)
    # (i, j) are not symmetric: a transposed index would change the words
    assert O.rng_bits(42, 1000, 0, 0, 1, 400, 400) != O.rng_bits(42, 1000, 0, 1, 0, 400, 400)
    # 64-bit wrap of seed + offset
    assert O.rng_bits(2**64 - 1, 1, 0, 0, 0, 4, 4) == O.rng_bits(0, 0, 0, 0, 0, 4, 4)


def test_c2_drop_count(O):
    keep = O.keep_mask(20, 400, 400, 0.2, 42, 1000)
    assert keep.size - int(keep.sum()) == 639_999


def _float_predicate_threshold_scan(p, T):
    """Over all 2^32 words: (float)w / 2^32 < p  <=>  w < T."""
    pf = np.float32(p)
    step = 1 << 26
    for lo in range(0, 1 << 32, step):
        w = np.arange(lo, lo + step, dtype=np.uint64).astype(np.uint32)
        pred = (w.astype(np.float32) / np.float32(4294967296.0)) < pf
        if not np.array_equal(pred, w.astype(np.uint64) < T):
            return False
    return True


@pytest.mark.parametrize("p", [0.1, 0.2])
def test_integer_threshold_exhaustive(pkg, p):
    T = pkg.drop_threshold(p)
    assert T == {0.1: 0x19999991, 0.2: 0x33333321}[p]
    assert T != int(np.floor(p * 2**32))  # the naive threshold is wrong
    assert _float_predicate_threshold_scan(p, T)


def test_integer_threshold_planted_mistake():
    """The exhaustive scan rejects the naive floor(p * 2^32) threshold."""
    assert not _float_predicate_threshold_scan(0.1, int(np.floor(0.1 * 2**32)))


@pytest.mark.parametrize("p", [1e-7, 1e-6, 0.05, 0.3, 0.5, 0.9, 0.999, 0.9999999])
def test_integer_threshold_boundaries(pkg, p):
    T = pkg.drop_threshold(p)
    pf = np.float32(p)
    u = lambda w: np.float32(w) / np.float32(4294967296.0)
    assert u(T) >= pf and (T == 0 or u(T - 1) < pf)


# ---------------------------------------------------------------------------
# attention math
# ---------------------------------------------------------------------------
def _load_tiny():
    z = np.load(os.path.join(GOLD, "tiny_attention.npz"), allow_pickle=False)
    names = sorted({k.split("__")[0] for k in z.files})
    return {n: {k.split("__")[1]: z[k] for k in z.files if k.startswith(n + "__")} for n in names}


@pytest.mark.parametrize("name", ["plain", "causal", "dropout", "causal_dropout"])
@pytest.mark.parametrize("gpu_gates", [False, True])
def test_oracle_matches_dense_fixture(O, name, gpu_gates):
    c = _load_tiny()[name]
    B, S_q, S_kv, D_qk, D_v, causal, seed, off = (int(x) for x in c["meta"])
    p, scale = float(c["p"][0]), float(c["p"][1])
    kw = dict(scale=scale, dropout=p, causal_mask=bool(causal), seed=seed, offset=off,
              gpu_gates=gpu_gates)
    keep = O.keep_mask(B, S_q, S_kv, p, seed, off) if p > 0 else np.ones_like(c["keep"])
    assert np.array_equal(keep, c["keep"])
    o, s = O.sdpa_fwd(c["q"], c["k"], c["v"], **kw)
    assert np.abs(o - c["o"]).max() < 2e-6
    assert np.abs(s - c["stats"]).max() < 2e-6
    dq, dk, dv = O.sdpa_bwd(c["q"], c["k"], c["v"], c["o"].astype(np.float32), s, c["d_o"], **kw)
    for got, ref in ((dq, c["dq"]), (dk, c["dk"]), (dv, c["dv"])):
        assert np.abs(got - ref).max() < 5e-6


def _fd_check(dense, c, grad_fn):
    """Central differences of L = sum(o * dO) for the dense float64 forward."""
    B, S_q, S_kv, D_qk, D_v, causal, seed, off = (int(x) for x in c["meta"])
    p, scale = float(c["p"][0]), float(c["p"][1])
    keep = c["keep"]
    q, k, v, d_o = (c[x].astype(np.float64) for x in ("q", "k", "v", "d_o"))

    def loss(q_, k_, v_):
        o, *_ = dense.dense_forward(q_, k_, v_, scale, bool(causal), p, keep)
        return float((o * d_o).sum())

    o, stats, P, Pd = dense.dense_forward(q, k, v, scale, bool(causal), p, keep)
    grads = grad_fn(q, k, v, o, d_o, scale, p, keep, P, Pd)
    h = 1e-6
    worst = 0.0
    for which, g in zip(range(3), grads):
        args = [q, k, v]
        x = args[which]
        it = np.nditer(x, flags=["multi_index"])
        for _ in it:
            idx = it.multi_index
            xp, xm = x.copy(), x.copy()
            xp[idx] += h
            xm[idx] -= h
            a_p, a_m = list(args), list(args)
            a_p[which], a_m[which] = xp, xm
            fd = (loss(*a_p) - loss(*a_m)) / (2 * h)
            worst = max(worst, abs(fd - g[idx]))
    return worst


@pytest.mark.parametrize("name", ["causal", "causal_dropout", "dropout"])
def test_dense_gradients_finite_difference(name):
    dense = golden_dense()
    c = _load_tiny()[name]
    assert _fd_check(dense, c, dense.dense_backward) < 1e-6


def test_finite_difference_catches_planted_mistakes():
    dense = golden_dense()
    c = _load_tiny()["causal_dropout"]

    def transposed_dk(q, k, v, o, d_o, scale, p, keep, P, Pd):
        dq, dk, dv = dense.dense_backward(q, k, v, o, d_o, scale, p, keep, P, Pd)
        dS = P * (np.einsum("bid,bjd->bij", d_o, v) * keep / (1 - p) - (d_o * o).sum(-1, keepdims=True))
        return dq, scale * np.einsum("bij,bjd->bid", dS, k).swapaxes(1, 1)[:, : k.shape[1]], dv

    def no_rescale(q, k, v, o, d_o, scale, p, keep, P, Pd):
        dq, dk, dv = dense.dense_backward(q, k, v, o, d_o, scale, p, keep, P, Pd)
        return dq, dk, dv * (1 - p)

    assert _fd_check(dense, c, transposed_dk) > 1e-3
    assert _fd_check(dense, c, no_rescale) > 1e-3


def test_oracle_invariants(O):
    rng = np.random.default_rng(1)
    B, S, D = 2, 37, 16
    k = rng.standard_normal((B, S, D)).astype(np.float32)
    v = rng.standard_normal((B, S, D)).astype(np.float32)
    q0 = np.zeros((B, S, D), np.float32)
    o, s = O.sdpa_fwd(q0, k, v, scale=0.25)
    assert np.abs(o - v.mean(axis=1, keepdims=True)).max() < 1e-6  # q = 0: mean of V
    assert np.allclose(s, np.log(np.float32(S) + np.float32(1e-6)), atol=1e-6)
    q = rng.standard_normal((B, S, D)).astype(np.float32)
    o, s = O.sdpa_fwd(q, k, v, scale=0.25, causal_mask=True)
    assert np.abs(o[:, 0] - v[:, 0]).max() < 1e-6  # causal row 0 sees only key 0
    # softmax rows sum to 1 (up to the 1e-6 in the statistic)
    sc = 0.25 * np.einsum("bid,bjd->bij", q.astype(np.float64), k.astype(np.float64))
    sc = np.where(np.triu(np.ones((S, S), bool), 1)[None], -np.inf, sc)
    assert np.allclose(np.exp(sc - s[..., None]).sum(-1), 1.0, atol=1e-5)


def test_fp16_faithful_close_to_gate(O):
    rng = np.random.default_rng(3)
    B, S, D = 2, 64, 32
    q, k, v, d_o = (rng.standard_normal((B, S, D)).astype(np.float16) for _ in range(4))
    kw = dict(scale=D ** -0.5, dropout=0.1, causal_mask=True, seed=9, offset=4)
    o16, s16 = O.sdpa_fwd(q, k, v, **kw)
    og, sg = O.sdpa_fwd_gate(q, k, v, **kw)
    assert np.abs(o16.astype(np.float32) - og.astype(np.float32)).max() < 5e-3
    assert np.abs(s16 - sg).max() < 5e-3
    g16 = O.sdpa_bwd(q, k, v, og, sg, d_o, accumulate_kv_in_t=True, **kw)
    gg = O.sdpa_bwd_gate(q, k, v, og, sg, d_o, **kw)
    for a, b in zip(g16, gg):
        assert np.abs(a.astype(np.float32) - b.astype(np.float32)).max() < 2e-2


def test_gpu_and_cpu_gates_differ_only_below_1e6(O):
    """p in (0, 1e-6] enables dropout on the CPU (sdpa_cpu.cc:274) but not on the
    GPU (sdpa_fwd.cu.cc:136); elsewhere the two gatings agree exactly."""
    rng = np.random.default_rng(5)
    q, k, v = (rng.standard_normal((2, 16, 8)).astype(np.float32) for _ in range(3))
    for p in (0.0, 0.3):
        a = O.sdpa_fwd(q, k, v, dropout=p, seed=1, offset=2, gpu_gates=True)
        b = O.sdpa_fwd(q, k, v, dropout=p, seed=1, offset=2, gpu_gates=False)
        assert np.array_equal(a[0], b[0]) and np.array_equal(a[1], b[1])
    a = O.sdpa_fwd(q, k, v, dropout=5e-7, seed=1, offset=2, gpu_gates=True)
    b = O.sdpa_fwd(q, k, v, dropout=5e-7, seed=1, offset=2, gpu_gates=False)
    assert not np.array_equal(a[0], b[0])  # CPU rescales by 1/(1-p) != 1


def _drop_all_closed_form(q, k, v, o, d_o, scale, causal):
    """float64 closed form of the reference with every element dropped
    (dropout > 1: u <= 1 < p; sdpa/sdpa_cpu.cc:274-285, 393-409):
    o = 0, stats as without dropout, dS = -P delta scale, dV = 0."""
    q, k, v, o, d_o = (a.astype(np.float64) for a in (q, k, v, o, d_o))
    s = scale * np.einsum("bid,bjd->bij", q, k)
    if causal:
        s = np.where(np.tril(np.ones(s.shape[1:], bool))[None], s, -np.inf)
    m = s.max(-1, keepdims=True)
    p = np.exp(s - m)
    l = p.sum(-1, keepdims=True)
    stats = (m + np.log(l + 1e-6))[..., 0]
    P = np.exp(s - stats[..., None])
    P = np.where(P < 1e-6, 0.0, P)                      # the backward's skip (sdpa_cpu.cc:384-385)
    delta = (d_o * o).sum(-1)                           # D_i (sdpa_cpu.cc:359-364)
    ds = -P * delta[..., None] * scale
    dq = np.einsum("bij,bjd->bid", ds, k)
    dk = np.einsum("bij,bid->bjd", ds, q)
    return stats, dq, dk, np.zeros(v.shape)


@pytest.mark.parametrize("gpu_gates", [True, False])
@pytest.mark.parametrize("causal", [False, True])
def test_oracle_dropout_above_one(O, gpu_gates, causal):
    """dropout > 1 drops every element in the reference: o = 0, stats as
    without dropout, dV = 0, dQ / dK from dS = -P delta.  The backward is run
    on an o that is not 0 (the reference takes o as given), so delta != 0."""
    rng = np.random.default_rng(5)
    B, S, Dq, Dv, scale = 2, 24, 16, 8, 0.3
    q, k = (rng.standard_normal((B, S, Dq)).astype(np.float32) for _ in range(2))
    v, o_in, d_o = (rng.standard_normal((B, S, Dv)).astype(np.float32) for _ in range(3))
    kw = dict(scale=scale, dropout=1.5, causal_mask=causal, seed=3, offset=9, gpu_gates=gpu_gates)
    o, s = O.sdpa_fwd(q, k, v, **kw)
    assert np.all(o == 0)
    stats, dq_ref, dk_ref, dv_ref = _drop_all_closed_form(q, k, v, o_in, d_o, scale, causal)
    assert np.abs(s - stats).max() < 1e-5
    _, s0 = O.sdpa_fwd(q, k, v, **dict(kw, dropout=0.0))
    assert np.abs(s - s0).max() == 0                   # l sums the undropped probabilities
    dq, dk, dv = O.sdpa_bwd(q, k, v, o_in, s, d_o, **kw)
    assert np.all(dv == 0)
    assert np.abs(dq - dq_ref).max() < 1e-5 and np.abs(dk - dk_ref).max() < 1e-5
    assert np.abs(dq).max() > 0.1                      # not trivially zero
