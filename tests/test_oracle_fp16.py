"""Pins the oracle's fp16-faithful mode (oracle/sdpa_oracle.cc, F16 element
semantics) before it is used as the reported fp16 CPU baseline:

* the two converters against numpy's IEEE binary16 (round to nearest even):
  half -> float exhaustively over all 65,536 patterns, float -> half on a
  sweep that holds every tie between two adjacent halves (normal, subnormal
  and the 65504 / inf boundary), the floats on either side of each tie, and
  every pattern of the float's top 19 bits with six low-bit endings;
* the half-rounded products of sdpa/sdpa_cpu.cc:261,363,378,424
  (static_cast<float>(Eigen::half * Eigen::half)) by closed-form cases whose
  exact and half-rounded answers differ by whole fp32 / fp16 ulps;
* the half read-modify-write of dK / dV (sdpa/sdpa_cpu.cc:416-417,437-438)
  by swamping: an accumulator at 2048 (fp16 ulp 2) does not move under
  increments below 1, where an fp32 accumulation does.

Each closed form is also run through a planted mistake -- the fp32
instantiation (no product rounding) or fp32 accumulation of dK / dV -- which
must fail it, and the converter sweep rejects a truncating converter.
"""
import numpy as np
import pytest


# ---------------------------------------------------------------------------
# converters
# ---------------------------------------------------------------------------
def test_half_to_float_exhaustive(O):
    h = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16)
    ref = h.view(np.float16).astype(np.float32)
    got = O.half_bits_to_float(h)
    nan = np.isnan(ref)
    assert np.array_equal(got.view(np.uint32)[~nan], ref.view(np.uint32)[~nan])
    assert np.isnan(got[nan]).all()
    # NaN payloads are carried over bit for bit (mantissa << 13, sign kept)
    nb = h[nan].astype(np.uint32)
    assert np.array_equal(got.view(np.uint32)[nan], ((nb & 0x8000) << 16) | 0x7F800000 | ((nb & 0x3FF) << 13))


def _sweep_floats():
    """float32 values around every rounding decision of float -> half."""
    # midpoints between adjacent finite halves (both signs), and the largest
    # finite half's midpoint towards infinity (65520)
    h = np.arange(0, 0x7C00, dtype=np.uint32).astype(np.uint16)
    lo = h.view(np.float16).astype(np.float64)
    hi = np.append(lo[1:], 65536.0)  # the "next" value above 65504 for rounding is 2^16
    mid = ((lo + hi) / 2).astype(np.float32)  # exact: a half midpoint needs <= 12 significant bits
    assert np.array_equal(mid.astype(np.float64), (lo + hi) / 2)
    mid_bits = mid.view(np.uint32)
    around = np.concatenate([mid_bits - 1, mid_bits, mid_bits + 1])
    # top 19 bits x low-13-bit endings (tie, just below / above, extremes)
    top = np.arange(1 << 19, dtype=np.uint32) << 13
    ends = np.array([0, 1, 0xFFF, 0x1000, 0x1001, 0x1FFF], dtype=np.uint32)
    grid = (top[:, None] | ends[None, :]).ravel()
    bits = np.concatenate([around, grid])
    bits = np.concatenate([bits, bits | 0x80000000])
    return bits.view(np.float32)


def _check_float_to_half(conv):
    f = _sweep_floats()
    with np.errstate(over="ignore"):
        ref = f.astype(np.float16).view(np.uint16)
    got = conv(f)
    nan = np.isnan(f)
    ok = np.array_equal(got[~nan], ref[~nan])
    # NaN -> quiet NaN 0x7e00 with the sign (Eigen's float_to_half_rtne)
    sign = ((f.view(np.uint32) >> 16) & 0x8000).astype(np.uint16)
    return ok and np.array_equal(got[nan], 0x7E00 | sign[nan])


def test_float_to_half_sweep(O):
    assert _check_float_to_half(O.float_to_half_bits)
    # spot values: ties to even, subnormals, overflow
    cases = {1.0 + 2.0 ** -11: 0x3C00, 1.0 + 3 * 2.0 ** -11: 0x3C02, 2.0 ** -24: 0x0001,
             2.0 ** -25: 0x0000, 1.5 * 2.0 ** -24: 0x0002, 65504.0: 0x7BFF, 65519.0: 0x7BFF,
             65520.0: 0x7C00, float("inf"): 0x7C00, -0.0: 0x8000}
    for x, want in cases.items():
        assert int(O.float_to_half_bits(np.array([x], np.float32))[0]) == want, x


def test_float_to_half_sweep_rejects_truncation():
    """Planted mistake: round-toward-zero instead of nearest-even."""
    def truncating(f):
        h = f.astype(np.float16)  # RNE, then step back one ulp where it rounded away from zero
        back = h.astype(np.float32)
        away = np.abs(back) > np.abs(f)
        hb = h.view(np.uint16).copy()
        hb[away & np.isfinite(f)] -= 1
        return hb
    with np.errstate(over="ignore", invalid="ignore"):
        assert not _check_float_to_half(truncating)


# ---------------------------------------------------------------------------
# half-rounded products (forward score, backward dP and delta)
# ---------------------------------------------------------------------------
E10 = 1.0 + 2.0 ** -10  # fp16-exact; E10 * E10 = 1 + 2^-9 + 2^-20, half-rounded to 1 + 2^-9


def _fwd_product_case(O, dtype):
    """D = 8, S = 1, q = k = E10: the score is 8 half(E10^2) = 8 + 2^-6 in the
    reference's fp16 kernel and 8 + 2^-6 + 2^-17 exactly.  One key: m = score,
    l = 1, stats = score + log(1 + 1e-6) (sdpa_cpu.cc:302)."""
    q = np.full((1, 1, 8), E10, dtype)
    _, s = O.sdpa_fwd(q, q.copy(), np.ones((1, 1, 4), dtype), scale=1.0, gpu_gates=False)
    return float(s[0, 0])


def test_fwd_half_product_rounding(O):
    tail = float(np.log(np.float32(1.0) + np.float32(1e-6)))
    want = float(np.float32(8.0 + 2.0 ** -6) + np.float32(tail))
    got = _fwd_product_case(O, np.float16)
    assert abs(got - want) <= 2 * 2.0 ** -20  # within 2 fp32 ulps at 8
    # planted mistake: the unrounded (fp32) product gives 8 more ulps
    unrounded = _fwd_product_case(O, np.float32)
    assert abs(unrounded - want) > 6 * 2.0 ** -20


def _bwd_product_case(O, dtype):
    """S = 1, D_qk = 1 (q = k = 1, scale 1, stats = 1 so P = exp(0) = 1),
    D_v = 8 with dO = V = E10 and O = 1:
      dP    = sum half(dO V)  = 8 (1 + 2^-9)     (exact: + 8 2^-20)
      delta = sum half(dO O)  = 8 (1 + 2^-10)    (exact, nothing rounded)
      dS    = P (dP - delta)  = 2^-7             (exact: 2^-7 + 2^-17)
    and dQ = dS k, dK = dS q, dV = P dO."""
    one = np.ones((1, 1, 1), dtype)
    v = np.full((1, 1, 8), E10, dtype)
    o = np.ones((1, 1, 8), dtype)
    stats = np.ones((1, 1), np.float32)
    return O.sdpa_bwd(one, one.copy(), v, o, stats, v.copy(), scale=1.0, gpu_gates=False,
                      accumulate_kv_in_t=(dtype == np.float16))


def test_bwd_half_product_rounding(O):
    dq, dk, dv = _bwd_product_case(O, np.float16)
    assert float(dq[0, 0, 0]) == 2.0 ** -7 and float(dk[0, 0, 0]) == 2.0 ** -7
    assert np.all(dv.astype(np.float32) == np.float32(E10))
    # planted mistake: unrounded products leave 2^-17, which fp16 keeps
    dq32, dk32, _ = _bwd_product_case(O, np.float32)
    assert float(np.float16(dq32[0, 0, 0])) == 2.0 ** -7 + 2.0 ** -17
    assert float(np.float16(dk32[0, 0, 0])) == 2.0 ** -7 + 2.0 ** -17


# ---------------------------------------------------------------------------
# half read-modify-write of dK / dV
# ---------------------------------------------------------------------------
def _swamp_case(O, dtype, kv_in_t, N=11):
    """S_q = N rows, one key, k = 0 (score 0, stats 0, P = 1), scale 1.
    dV_0[1] = sum_i P dO_i[1] with dO_0[1] = 2048, dO_i[1] = 0.9:  in half
    each 0.9 is below half an ulp of 2048, so the RMW stays at 2048; in fp32
    it reaches 2048 + 0.9 (N - 1) = 2056.9 (2056 in fp16).
    dK_0 = sum_i dS_i q_i with V_0 = e_0, dO_i[0] = 1 and O = 0, so
    dP_i = 1, delta_i = 0 and dS_i = 1; q_0 = 2048, q_i = 0.9 swamps the same
    way."""
    D = 2
    q = np.zeros((1, N, 1), dtype)
    q[0, 0, 0], q[0, 1:, 0] = 2048.0, 0.9
    k = np.zeros((1, 1, 1), dtype)
    v = np.zeros((1, 1, D), dtype)
    v[0, 0, 0] = 1.0
    d_o = np.zeros((1, N, D), dtype)
    d_o[0, :, 0] = 1.0        # dP_i = dO_i . V_0 = 1
    d_o[0, 0, 1] = 2048.0     # dV_0[1] = 2048 + 0.9 (N - 1) in fp32
    d_o[0, 1:, 1] = 0.9
    o = np.zeros((1, N, D), dtype)  # delta_i = 0, so dS_i = P dP_i = 1
    stats = np.zeros((1, N), np.float32)
    return O.sdpa_bwd(q, k, v, o, stats, d_o, scale=1.0, gpu_gates=False,
                      accumulate_kv_in_t=kv_in_t)


def test_half_rmw_swamping(O):
    dq, dk, dv = _swamp_case(O, np.float16, True)
    assert float(dv[0, 0, 1]) == 2048.0  # 0.9 < ulp/2 each time: stalls
    assert float(dv[0, 0, 0]) == 11.0    # small increments of 1 are exact
    assert float(dk[0, 0, 0]) == 2048.0  # dS_i q_i: 2048, then 0.9s that vanish
    assert np.all(dq == 0)               # dQ_i = dS_i k = 0


def test_half_rmw_swamping_planted_mistake(O):
    """fp32 accumulation of dK / dV (rounded once at the end) moves on."""
    _, dk, dv = _swamp_case(O, np.float16, False)
    assert float(dv[0, 0, 1]) == 2056.0 and float(dk[0, 0, 0]) == 2056.0


# ---------------------------------------------------------------------------
# output rounding and row ranges
# ---------------------------------------------------------------------------
def test_fwd_output_rounding(O):
    """o = half(acc * inv_l), one rounding of the fp32 value (sdpa_cpu.cc:308).
    One key: l = 1 and o = V bit for bit.  Two keys of equal score with
    v0 = 1, v1 = 2^-11: acc = 1 + 2^-11 (fp32-exact), o = 0.5 + 2^-12, a tie
    that rounds to the even 0.5; with v1 = 3 2^-11 the tie 0.5 + 3 2^-12
    rounds up to 0.5 + 2^-10."""
    rng = np.random.default_rng(0)
    v = rng.standard_normal((2, 1, 16)).astype(np.float16)
    q = rng.standard_normal((2, 3, 4)).astype(np.float16)
    k = rng.standard_normal((2, 1, 4)).astype(np.float16)
    o, _ = O.sdpa_fwd(q, k, v, scale=0.5, gpu_gates=False)
    assert np.array_equal(o, np.broadcast_to(v, o.shape))
    q0 = np.zeros((1, 1, 4), np.float16)
    k0 = np.zeros((1, 2, 4), np.float16)
    for v1, want in ((2.0 ** -11, 0.5), (3 * 2.0 ** -11, 0.5 + 2.0 ** -10)):
        v2 = np.array([[[1.0], [v1]]], np.float16)
        o2, _ = O.sdpa_fwd(q0, k0, v2, scale=1.0, gpu_gates=False)
        assert float(o2[0, 0, 0]) == want


@pytest.mark.parametrize("dtype", [np.float32, np.float16])
def test_row_range_matches_full_run(O, dtype):
    """rows=(i0, i1) computes exactly those rows of the full computation."""
    rng = np.random.default_rng(4)
    q, k, v, d_o = (rng.standard_normal((3, 40, 16)).astype(dtype) for _ in range(4))
    kw = dict(scale=0.25, dropout=0.2, causal_mask=True, seed=3, offset=99)
    o, s = O.sdpa_fwd(q, k, v, **kw)
    o2, s2 = O.sdpa_fwd(q, k, v, rows=(10, 25), **kw)
    assert np.array_equal(o2[:, 10:25], o[:, 10:25]) and np.array_equal(s2[:, 10:25], s[:, 10:25])
    o3, s3 = O.sdpa_fwd(q, k, v, rows=(3, 40, 7), **kw)
    assert np.array_equal(o3[:, 3::7], o[:, 3::7]) and np.array_equal(s3[:, 3::7], s[:, 3::7])
    dq, dk, dv = O.sdpa_bwd(q, k, v, o, s, d_o, **kw)
    dq2, _, _ = O.sdpa_bwd(q, k, v, o, s, d_o, rows=(10, 25), **kw)
    assert np.array_equal(dq2[:, 10:25], dq[:, 10:25])
    dq3, _, _ = O.sdpa_bwd(q, k, v, o, s, d_o, rows=(2, 40, 5), **kw)
    assert np.array_equal(dq3[:, 2::5], dq[:, 2::5])
    _, dk4, dv4 = O.sdpa_bwd(q, k, v, o, s, d_o, keys=(1, 40, 6), **kw)
    assert np.array_equal(dk4[:, 1::6], dk[:, 1::6]) and np.array_equal(dv4[:, 1::6], dv[:, 1::6])
