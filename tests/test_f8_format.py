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
