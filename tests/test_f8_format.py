"""The numpy model of the VSL_DT_F16F8 form that the GPU tests check the kernels against (CPU): e4m3
decoding, round-to-nearest-even encoding, saturation, the lo plane's byte order, and the accuracy the
form carries -- pinned by closed forms and exhaustive checks, not by re-deriving the same formulas."""
import numpy as np

import vsl_testlib as T


def test_e4m3_table_known_codes():
    t = T.e4m3_table()
    known = {0x00: 0.0, 0x01: 2.0 ** -9, 0x07: 7 * 2.0 ** -9, 0x08: 2.0 ** -6, 0x38: 1.0, 0x39: 1.125,
             0x40: 2.0, 0x7E: 448.0, 0xB8: -1.0, 0xFE: -448.0}
    for c, v in known.items():
        assert t[c] == v, hex(c)
    assert np.signbit(t[0x80]) and t[0x80] == 0.0
    assert np.isnan(t[0x7F]) and np.isnan(t[0xFF])
    # 126 distinct positive finite values, increasing with the code
    assert np.all(np.diff(t[:127]) > 0)


def test_e4m3_encode_exhaustive():
    t = T.e4m3_table()
    finite = np.array([c for c in range(256) if c not in (0x7F, 0xFF)])
    assert np.array_equal(T.e4m3_encode(t[finite]), finite.astype(np.uint8))
    # every midpoint between neighbours goes to the even code; a nudge either way decides
    pos = t[:127]
    mid = (pos[:-1] + pos[1:]) / 2
    codes = T.e4m3_encode(mid)
    want = np.where(np.arange(126) % 2 == 0, np.arange(126), np.arange(1, 127))
    assert np.array_equal(codes, want)
    assert np.array_equal(T.e4m3_encode(np.nextafter(mid, 0)), np.arange(126))
    assert np.array_equal(T.e4m3_encode(np.nextafter(mid, 1e9)), np.arange(1, 127))
    # saturation and signed zeros
    assert list(T.e4m3_encode([448.0, 1e6, -1e6, 0.0, -0.0, -1e-12])) == [0x7E, 0x7E, 0xFE, 0x00, 0x80, 0x80]


def test_lo8_order_feeds_lane_groups():
    """Column 16 t + 8 g + e (t = 0, 1; e = 0..7) of every 32-column block sits at byte 16 g + 8 t + e:
    lane group g of the fp8 MFMA reads one contiguous 16-byte chunk. The order is its own inverse."""
    p = T.lo8_perm(128)
    for blk in range(4):
        for g in range(2):
            for t in range(2):
                for e in range(8):
                    assert p[32 * blk + 16 * t + 8 * g + e] == 32 * blk + 16 * g + 8 * t + e
    assert np.array_equal(p[p], np.arange(128))
    # groups of four columns stay contiguous and in order (four-value stores)
    assert np.all(np.diff(p.reshape(-1, 4), axis=1) == 1)


def test_f16f8_split_accuracy():
    """hi is the binary16 rounding; for |v| <= 224 (where |v - hi| 2^12 <= 2 |v| stays within e4m3's
    448) hi + lo8 2^-12 is within 2^-16 relative of the fp32 value, plus the subnormal floor 2^-22 for
    tiny remainders, ~16x closer than hi alone on average; above that the clamped remainder still
    moves hi toward v (never further away)."""
    rng = np.random.default_rng(0)
    a = (rng.normal(0, 1, (64, 256)) * np.exp(rng.normal(0, 2, (64, 256)))).astype(np.float32)
    hi, plane, val = T.f16f8_split(a)
    assert np.array_equal(hi, a.astype(np.float16))
    assert np.array_equal(T.f16f8_value(hi, plane), val)
    err = np.abs(val - a.astype(np.float64))
    e16 = np.abs(hi.astype(np.float64) - a)
    small = np.abs(a) <= 224
    assert small.mean() > 0.9 and (~small).sum() > 10
    assert np.all(err[small] <= 2.0 ** -16 * np.abs(a[small]) + 2.0 ** -22)
    assert np.mean(err[small]) * 16 < np.mean(e16[small])
    assert np.all(err[~small] <= e16[~small])


def test_f8lo_product_model():
    """The GEMM model: the lo term uses B rounded to e4m3 at scale 2^6 -- exact for weights that are
    e4m3 values / 64 already, so the model then equals the plain product of the carried values."""
    rng = np.random.default_rng(1)
    t = T.e4m3_table()
    codes = rng.integers(0, 126, (16, 64))
    B = (t[codes] * np.where(rng.random((16, 64)) < 0.5, -1, 1) / 64.0).astype(np.float16)
    a = rng.normal(0, 1, (8, 64)).astype(np.float32)
    hi, plane, val = T.f16f8_split(a)
    got = T.f8lo_product(hi, val - hi.astype(np.float64), B)
    assert np.allclose(got, val @ B.astype(np.float64).T, rtol=0, atol=1e-12)


def test_b8_shift_closed_form(vsl):
    """vsl_gemm_b8_shift (host arithmetic): the largest shift that keeps max_abs * 2^s within e4m3's 448,
    against a search over every shift and against values worked out by hand: 7 * 2^6 = 448 exactly,
    7.5 and 40 need 5 and 3, fp16's largest 65504 needs -8, N(0, 0.02) weights (max ~0.1) get 11."""
    H = vsl.hip()
    hand = {7.0: 6, 7.5: 5, 40.0: 3, 448.0: 0, 448.5: -1, 65504.0: -8, 0.1: 12, 0.109: 12, 0.11: 11,
            1.0: 8, 1e-30: 30, 0.0: 6, float("inf"): 6, float("nan"): 6, -3.0: 6}
    for m, s in hand.items():
        assert H.vsl_gemm_b8_shift(m) == s, m
        assert T.b8_shift_model(m) == s, m
    rng = np.random.default_rng(5)
    vals = np.concatenate([np.exp(rng.uniform(-20, 12, 2000)), T.e4m3_table()[1:127] / 64.0,
                           np.ldexp(448.0, -np.arange(0, 30))]).astype(np.float32)
    for m in vals:
        s = H.vsl_gemm_b8_shift(float(m))
        assert s == T.b8_shift_model(m), m
        assert np.ldexp(np.float64(m), s) <= 448.0 and (s == 30 or np.ldexp(np.float64(m), s + 1) > 448.0)


def test_f8lo_product_shift_is_exact_scaling():
    """With every |B| 2^s <= 448 the model's e4m3 rounding of B never saturates, and a different shift
    changes B8 only by the subnormal floor: two shifts 4 apart agree wherever |B| 2^s stays normal."""
    rng = np.random.default_rng(2)
    B = rng.normal(0, 0.5, (8, 64)).astype(np.float16)
    B[0, :4] = [40.0, -7.5, 100.0, -300.0]
    a = rng.normal(0, 1, (4, 64)).astype(np.float32)
    hi, plane, val = T.f16f8_split(a)
    s = T.b8_shift_model(np.max(np.abs(B.astype(np.float32))))
    assert s == 0
    lo = val - hi.astype(np.float64)
    p0 = T.f8lo_product(hi, lo, B, s)
    assert np.all(np.isfinite(p0))
    B8 = np.ldexp(T.e4m3_table()[T.e4m3_encode(np.ldexp(B.astype(np.float64), s))], -s)
    assert np.all(np.abs(B8 - B) <= 2.0 ** -4 * np.abs(B) + np.ldexp(2.0 ** -10, -s))
    normal = np.abs(np.ldexp(B.astype(np.float64), s - 4)) >= 2.0 ** -6
    B8b = np.ldexp(T.e4m3_table()[T.e4m3_encode(np.ldexp(B.astype(np.float64), s - 4))], 4 - s)
    assert np.array_equal(B8[normal], B8b[normal])
