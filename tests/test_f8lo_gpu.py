"""The VSL_DT_F16F8 activation form on the GPU: producers (row RMSNorm, the fused residual + RMSNorm,
the SwiGLU epilogue) against the fp64 value they encode, and the GEMM's fp8 lo path against the
product it is defined to compute -- hi B^T + lo B8^T with lo the e4m3 plane's value and B8 the e4m3
rounding of B * 2^6 -- in float64 (vsl_testlib.f8lo_product), through the big / mid tiles, the K
split, and the forced direct-to-LDS path for shapes that would otherwise take another kernel."""
import numpy as np
import pytest

import vsl_testlib as T

pytestmark = pytest.mark.gpu

F8_VALUE_REL = 2.0 ** -16   # |hi + lo8 2^-12 - v| / |v| for normal lo (e4m3 rounds to 2^-4 of lo <= 2^-12 v)
F8_VALUE_ABS = 2.0 ** -22   # e4m3 subnormal spacing 2^-9, times 2^-12, halved


@pytest.fixture(scope="module")
def _dev():
    return T.Dev()


@pytest.fixture
def dev(_dev):
    yield _dev
    _dev.release()


@pytest.fixture(scope="module")
def H(vsl):
    return vsl.hip()


def ok(vsl, rc):
    vsl.check(rc)


def rel_err(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.max(np.abs(a - b)) / max(1e-30, np.max(np.abs(b))))


def f8_buffer(dev, a):
    """Device VSL_DT_F16F8 copy of fp32 rows a: the hi plane, then the byte plane. Returns (buffer,
    hi, value)."""
    hi, plane, val = T.f16f8_split(a)
    buf = dev.put(np.concatenate([hi.reshape(-1).view(np.uint8), plane.reshape(-1)]))
    return buf, hi, val


def f8_read(dev, buf, M, N):
    """(hi, value) of a device VSL_DT_F16F8 buffer of M x N."""
    flat = dev.get(buf).reshape(-1).view(np.uint8)
    hi = flat[:2 * M * N].view(np.float16).reshape(M, N)
    plane = flat[2 * M * N:3 * M * N].reshape(M, N)
    return hi, T.f16f8_value(hi, plane)


def assert_f8_encodes(hi, val, ref):
    """hi is the binary16 rounding of the encoded value's fp32 source and hi + lo8 2^-12 carries it
    to e4m3's precision: within 2^-16 relative plus the subnormal floor, element by element."""
    ref = np.asarray(ref, np.float64)
    err = np.abs(val - ref)
    assert np.all(err <= F8_VALUE_REL * np.abs(ref) + F8_VALUE_ABS + 4e-7 * np.abs(ref)), float(np.max(err))
    assert np.all(np.abs(hi.astype(np.float64) - ref) <= np.spacing(np.abs(hi)).astype(np.float64))


@pytest.mark.parametrize("d", [256, 2048, 4096, 8192, 1056])
@pytest.mark.parametrize("rows", [1, 6])
def test_rmsnorm_f16f8(vsl, orc, dev, H, d, rows):
    """Row RMSNorm into the F16F8 form: the one-row-per-wave kernel (256 .. 8192) and the block-per-row
    kernel (1056); every element's hi + lo8 2^-12 is the oracle's RMSNorm to e4m3 precision of the
    remainder (a byte in the wrong position of the plane misses that by ~2^-12)."""
    rng = np.random.default_rng(d + rows)
    x = rng.normal(0, 2, (rows, d)).astype(np.float32)
    g = rng.normal(1, 0.1, d).astype(np.float32)
    out = dev.empty((3 * rows * d,), np.uint8)
    ok(vsl, H.vsl_rmsnorm(dev.p(dev.put(x)), dev.p(dev.put(g)), rows, d, 1e-5, dev.p(out), vsl.VSL_DT_F16F8, None))
    hi, val = f8_read(dev, out, rows, d)
    ref = np.stack([orc.rmsnorm(x[r], g, 1e-5) for r in range(rows)]).astype(np.float64)
    assert_f8_encodes(hi, val, ref)


def test_rmsnorm_f16f8_needs_whole_blocks(vsl, dev, H):
    x = dev.put(np.ones((2, 1000), np.float32))
    out = dev.empty((6000,), np.uint8)
    assert H.vsl_rmsnorm(dev.p(x), None, 2, 1000, 1e-5, dev.p(out), vsl.VSL_DT_F16F8, None) == vsl.VSL_E_INVALID


@pytest.mark.parametrize("M,N,K,epi,amode", [
    (128, 8192, 640, 3, "x2"),      # SwiGLU, hi/lo fp16 A: 2 x 128 tiles of 64 x (64 + 64), 10 stages of 64
    (128, 16384, 896, 0, "x2"),     # fp32 store, hi/lo fp16 A, 14 stages
    (128, 16384, 384, 0, "f8"),     # fp32 store, F16F8 A, 6 stages
    (128, 8192, 640, 3, "f8"),      # SwiGLU, F16F8 A
    (100, 8192, 1152, 3, "one"),    # one fp16 plane (32-column stages), ragged M
])
def test_gemm_small_tiles_odd_k_stages(vsl, dev, H, M, N, K, epi, amode):
    """The 64 x 128 direct-to-LDS tiles run the split-A and fp8-lo forms with four 64-column stage
    buffers; K an odd multiple of 128 leaves a last pair of stages after the four-stage rounds, which
    must be multiplied once each (rows 0, M-1 and a sample against the fp64 product of what the form
    carries)."""
    rng = np.random.default_rng(M + N + K + epi)
    nb = 2 * N if epi == 3 else N
    A = rng.normal(0, 1, (M, K)).astype(np.float32)
    B = rng.normal(0, 0.02, (nb, K)).astype(np.float16)
    rows = np.unique(np.concatenate([[0, M - 1, M // 2], rng.integers(0, M, 24)]))
    if amode == "f8":
        dA, hi, val = f8_buffer(dev, A)
        prod = T.f8lo_product(hi[rows], val[rows] - hi[rows].astype(np.float64), B)
        flags = vsl.GEMM_A_F8
    elif amode == "x2":
        hi = A.astype(np.float16)
        lo = (A - hi.astype(np.float32)).astype(np.float16)
        dA = dev.put(np.concatenate([hi, lo]))
        prod = (hi[rows].astype(np.float64) + lo[rows].astype(np.float64)) @ B.astype(np.float64).T
        flags = vsl.GEMM_A_X2
    else:
        a16 = A.astype(np.float16)
        dA = dev.put(a16)
        prod = a16[rows].astype(np.float64) @ B.astype(np.float64).T
        flags = 0
    C = dev.empty((M, N), np.float16 if epi == 3 else np.float32)
    ok(vsl, H.vsl_gemm_f16(dev.p(dA), dev.p(dev.put(B)), M, N, K, dev.p(C), epi | flags, None))
    out = dev.get(C).astype(np.float64)[rows]
    if epi == 3:
        ref = prod[:, :N] / (1.0 + np.exp(-prod[:, :N])) * prod[:, N:]
        assert rel_err(out, ref) < 2.0 ** -10
    else:
        assert rel_err(out, prod) < 1e-5


@pytest.mark.parametrize("M,N,K,epi,cmode", [
    (512, 14336, 2048, 3, "f8"),    # SwiGLU, 256 x 256 tiles, F16F8 output
    (512, 14336, 2048, 3, "x2"),    # F16F8 in, hi/lo fp16 out
    (700, 14336, 1024, 3, "f8"),    # ragged M on the 256 x 256 tiles (rows 512..699 in the last tile)
    (777, 4096, 2048, 3, "f16"),    # ragged M on 128 x 256 tiles, fp16 out
    (777, 4096, 2048, 3, "f8"),
    (2048, 6144, 4096, 0, None),    # fp32 store, 256 x 256
    (2048, 4096, 1024, 2, None),    # residual add, 128 x 256 (16 x 16 tiles)
    (1536, 8192, 256, 1, None),     # fp16 store, two 128-column stage groups
])
def test_gemm_f8lo_tiles(vsl, dev, H, M, N, K, epi, cmode):
    rng = np.random.default_rng(M + N + K + epi)
    nb = 2 * N if epi == 3 else N
    A = rng.normal(0, 1, (M, K)).astype(np.float32)
    B = rng.normal(0, 0.02, (nb, K)).astype(np.float16)
    dA, hi, val = f8_buffer(dev, A)
    lo = val - hi.astype(np.float64)
    flags = vsl.GEMM_A_F8 | {"f8": vsl.GEMM_C_F8, "x2": vsl.GEMM_C_X2, "f16": 0, None: 0}[cmode]
    if epi == 3:
        C = dev.empty((4 * M * N,), np.uint8)
    elif epi == 1:
        C = dev.empty((M, N), np.float16)
    else:
        C0 = rng.normal(0, 1, (M, N)).astype(np.float32) if epi == 2 else np.zeros((M, N), np.float32)
        C = dev.put(C0)
    ok(vsl, H.vsl_gemm_f16(dev.p(dA), dev.p(dev.put(B)), M, N, K, dev.p(C), epi | flags, None))
    rows = np.unique(np.concatenate([[0, M - 1, M // 2], rng.integers(0, M, 40)]))
    prod = T.f8lo_product(hi[rows], lo[rows], B)
    exact = A[rows].astype(np.float64) @ B.astype(np.float64).T
    if epi == 3:
        g, u = prod[:, :N], prod[:, N:]
        ref = g / (1.0 + np.exp(-g)) * u
        flat = dev.get(C).reshape(-1).view(np.uint8)
        if cmode == "f8":
            hi_o = flat[:2 * M * N].view(np.float16).reshape(M, N)
            got = T.f16f8_value(hi_o[rows], flat[2 * M * N:3 * M * N].reshape(M, N)[rows])
            assert rel_err(got, ref) < 2.0 ** -15  # the output form itself carries 2^-16 of each value
            assert rel_err(hi_o[rows], ref) < 2.0 ** -11
        elif cmode == "x2":
            o = flat[:4 * M * N].view(np.float16).reshape(2, M, N).astype(np.float64)
            got = o[0, rows] + o[1, rows]
            assert rel_err(got, ref) < 2e-6
        else:
            got = flat[:2 * M * N].view(np.float16).reshape(M, N)[rows].astype(np.float64)
            assert rel_err(got, ref) < 2.0 ** -10
        ge, ue = exact[:, :N], exact[:, N:]
        assert rel_err(got, ge / (1.0 + np.exp(-ge)) * ue) < (2.0 ** -10 if cmode == "f16" else 2.0 ** -12)
    else:
        out = dev.get(C).astype(np.float64)[rows]
        if epi == 1:
            assert rel_err(out, prod) < 2.0 ** -10
        else:
            base = C0[rows] if epi == 2 else 0.0
            assert rel_err(out - base, prod) < 5e-6
            # ~15-bit inputs: far closer to the fp32-input product than one fp16 rounding (2^-11)
            assert rel_err(out - base, exact) < 2.0 ** -13


@pytest.mark.parametrize("M,N,K,epi", [
    (512, 4096, 14336, 2),   # 8B down projection of a 512-row chunk
    (512, 6144, 4096, 0),    # 8B QKV (128 x 192 tiles)
    (128, 2048, 8192, 2),    # 1B down projection of a 128-row prompt: 32 chunks
    (300, 4096, 2048, 1),    # ragged M, fp16 store
])
def test_gemm_f8lo_splitk(vsl, dev, H, M, N, K, epi):
    """Narrow shapes split over K with an F16F8 A: the partials come from the fp8 lo path of the
    128 x 256 tiles (128 x 192 for the QKV width); without the workspace the direct-to-LDS tiles (64 x
    128 where they give 192 tiles, else the larger ones at lower occupancy) give the same result (to
    fp32 rounding of the accumulation order)."""
    rng = np.random.default_rng(3 * M + N + K + epi)
    A = rng.normal(0, 1, (M, K)).astype(np.float32)
    B = rng.normal(0, 0.02, (N, K)).astype(np.float16)
    dA, hi, val = f8_buffer(dev, A)
    flags = epi | vsl.GEMM_A_F8
    need = H.vsl_gemm_f16_ws_bytes(M, N, K, flags)
    assert need > 0
    ws = dev.empty((need // 4 + 4,), np.float32)
    C0 = rng.normal(0, 1, (M, N)).astype(np.float32) if epi == 2 else np.zeros((M, N), np.float32)
    rows = np.unique(np.concatenate([[0, M - 1], rng.integers(0, M, 40)]))
    ref = T.f8lo_product(hi[rows], val[rows] - hi[rows].astype(np.float64), B)
    for with_ws in (True, False):
        C = dev.empty((M, N), np.float16) if epi == 1 else dev.put(C0)
        if with_ws:
            ok(vsl, H.vsl_gemm_f16_ws(dev.p(dA), dev.p(dev.put(B)), M, N, K, dev.p(C), flags, dev.p(ws), need, None))
        else:
            ok(vsl, H.vsl_gemm_f16(dev.p(dA), dev.p(dev.put(B)), M, N, K, dev.p(C), flags, None))
        out = dev.get(C).astype(np.float64)[rows]
        if epi == 1:
            assert rel_err(out, ref) < 2.0 ** -10
        else:
            assert rel_err(out - (C0[rows] if epi == 2 else 0.0), ref) < 5e-6


@pytest.mark.parametrize("n,off", [(1, 0), (7, 0), (8, 0), (1000, 1), (4097, 3), (1 << 20, 0), ((1 << 20) + 5, 8)])
def test_absmax_f16(vsl, dev, H, n, off):
    """vsl_absmax_f16: the largest finite |x| (infinities and NaN skipped) over any length and start
    (16-byte aligned or not), folded into the value already there."""
    rng = np.random.default_rng(n + off)
    x = rng.normal(0, 1, n + off).astype(np.float16)
    if n > 16:
        x[off + rng.integers(0, n, 3)] = [np.inf, -np.inf, np.nan]
        x[off + rng.integers(0, n)] = np.float16(-3000.0)
    body = x[off:].astype(np.float32)
    want = float(np.max(np.abs(body[np.isfinite(body)]))) if np.any(np.isfinite(body)) else 0.0
    buf = dev.put(x)
    base = dev.p(buf) + 2 * off
    out = dev.put(np.zeros(1, np.float32))
    ok(vsl, H.vsl_absmax_f16(base, n, dev.p(out), None))
    assert float(dev.get(out)[0]) == want
    out2 = dev.put(np.array([want * 2 + 1], np.float32))
    ok(vsl, H.vsl_absmax_f16(base, n, dev.p(out2), None))
    assert float(dev.get(out2)[0]) == want * 2 + 1


def _weights(kind, rows, K, rng):
    """fp16 weights of a range scenario: N(0, 0.002), N(0, 0.2), or N(0, 0.02) with planted outliers."""
    if kind == "std0.002":
        return rng.normal(0, 0.002, (rows, K)).astype(np.float16)
    if kind == "std0.2":
        return rng.normal(0, 0.2, (rows, K)).astype(np.float16)
    B = rng.normal(0, 0.02, (rows, K)).astype(np.float16)
    big = {"out40": [7.5, -7.5, 40.0, -40.0], "out1000": [7.5, -40.0, 100.0, -1000.0]}[kind]
    idx = rng.choice(rows * K, 64, replace=False)
    B.reshape(-1)[idx] = np.resize(np.array(big, np.float16), 64)
    return B


@pytest.mark.parametrize("kind", ["std0.002", "std0.2", "out40", "out1000"])
@pytest.mark.parametrize("M,N,K,epi,ks", [
    (1536, 8192, 1024, 3, False),   # SwiGLU on 256 x 256 tiles
    (512, 4096, 1024, 3, False),    # SwiGLU on 64 x 128 tiles
    (2048, 4096, 1024, 2, False),   # residual on 128 x 256 tiles
    (512, 4096, 4096, 2, True),     # K split on 128 x 256 tiles
    (512, 6144, 4096, 0, True),     # K split on 128 x 192 tiles
])
def test_gemm_f8lo_weight_ranges(vsl, dev, H, kind, M, N, K, epi, ks):
    """The fp8 lo product over weight ranges other than N(0, 0.02): small (std 0.002), wide (std 0.2) and
    planted outliers up to 40 or 1000. The shift from vsl_absmax_f16 + vsl_gemm_b8_shift keeps every
    weight within e4m3's range: the result is finite, equals the model of hi B^T + lo e4m3(B 2^s) 2^-s,
    and stays within one fp16 rounding of the fp32-input product (much closer without outliers)."""
    rng = np.random.default_rng(M + N + K + epi + len(kind))
    nb = 2 * N if epi == 3 else N
    A = rng.normal(0, 1, (M, K)).astype(np.float32)
    B = _weights(kind, nb, K, rng)
    dB = dev.put(B)
    mx = dev.put(np.zeros(1, np.float32))
    ok(vsl, H.vsl_absmax_f16(dev.p(dB), nb * K, dev.p(mx), None))
    amax = float(dev.get(mx)[0])
    assert amax == float(np.max(np.abs(B.astype(np.float32))))
    s = H.vsl_gemm_b8_shift(amax)
    assert s == T.b8_shift_model(amax)
    dA, hi, val = f8_buffer(dev, A)
    lo = val - hi.astype(np.float64)
    # SwiGLU writes hi/lo fp16 planes (~22 bits, no clamped remainder however large the outputs grow)
    flags = epi | vsl.GEMM_A_F8 | vsl.GEMM_B8_SHIFT(s) | (vsl.GEMM_C_X2 if epi == 3 else 0)
    if epi == 3:
        C = dev.empty((4 * M * N,), np.uint8)
    else:
        C0 = rng.normal(0, 1, (M, N)).astype(np.float32) if epi == 2 else np.zeros((M, N), np.float32)
        C = dev.put(C0)
    if ks:
        need = H.vsl_gemm_f16_ws_bytes(M, N, K, flags)
        assert need > 0
        ws = dev.empty((need // 4 + 4,), np.float32)
        ok(vsl, H.vsl_gemm_f16_ws(dev.p(dA), dev.p(dB), M, N, K, dev.p(C), flags, dev.p(ws), need, None))
    else:
        ok(vsl, H.vsl_gemm_f16(dev.p(dA), dev.p(dB), M, N, K, dev.p(C), flags, None))
    rows = np.unique(np.concatenate([[0, M - 1], rng.integers(0, M, 40)]))
    prod = T.f8lo_product(hi[rows], lo[rows], B, s)
    exact = A[rows].astype(np.float64) @ B.astype(np.float64).T
    bound = 2.0 ** -11 if kind == "out1000" else 2.0 ** -13
    if epi == 3:
        o = dev.get(C).reshape(-1).view(np.uint8)[:4 * M * N].view(np.float16).reshape(2, M, N).astype(np.float64)
        got = o[0, rows] + o[1, rows]
        assert np.all(np.isfinite(got))
        g, u = prod[:, :N], prod[:, N:]
        assert rel_err(got, g / (1.0 + np.exp(-g)) * u) < 5e-6
        ge, ue = exact[:, :N], exact[:, N:]
        assert rel_err(got, ge / (1.0 + np.exp(-ge)) * ue) < bound
    else:
        out = dev.get(C).astype(np.float64)[rows] - (C0[rows] if epi == 2 else 0.0)
        assert np.all(np.isfinite(out))
        assert rel_err(out, prod) < 5e-6
        assert rel_err(out, exact) < bound


def test_gemm_f8lo_default_shift_is_not_saturating(vsl, dev, H):
    """Why the shift exists: at the default 2^6 a weight of 40 becomes 2560, past e4m3's 448, and the
    conversion does not saturate -- the output columns of that weight's row are not finite, every other
    column is the model's. With the measured shift all columns are."""
    rng = np.random.default_rng(9)
    M, N, K = 2048, 4096, 1024
    A = rng.normal(0, 1, (M, K)).astype(np.float32)
    B = rng.normal(0, 0.02, (N, K)).astype(np.float16)
    B[[5, 300], [17, 900]] = [40.0, -40.0]
    dA, hi, val = f8_buffer(dev, A)
    lo = val - hi.astype(np.float64)
    dB = dev.put(B)
    rows = np.arange(0, M, 97)
    for shift in (None, 3):
        C = dev.put(np.zeros((M, N), np.float32))
        flags = 2 | vsl.GEMM_A_F8 | (vsl.GEMM_B8_SHIFT(shift) if shift is not None else 0)
        ok(vsl, H.vsl_gemm_f16(dev.p(dA), dev.p(dB), M, N, K, dev.p(C), flags, None))
        out = dev.get(C).astype(np.float64)[rows]
        cols = np.setdiff1d(np.arange(N), [5, 300])
        ref = T.f8lo_product(hi[rows], lo[rows], B, 6 if shift is None else shift)
        assert rel_err(out[:, cols], ref[:, cols]) < 5e-6
        if shift is None:
            assert not np.any(np.isfinite(out[:, [5, 300]]))
        else:
            assert np.all(np.isfinite(out)) and rel_err(out, ref) < 5e-6


def test_gemm_b8_shift_flags_refused(vsl, dev, H):
    A = dev.put(np.zeros((3 * 64 * 4096,), np.uint8))
    B = dev.put(np.zeros((4096, 4096), np.float16))
    C = dev.put(np.zeros((64, 4096), np.float32))
    for s in (vsl.GEMM_B8_SHIFT(-17), vsl.GEMM_B8_SHIFT(31)):
        assert H.vsl_gemm_f16(dev.p(A), dev.p(B), 64, 4096, 4096, dev.p(C), vsl.GEMM_A_F8 | s, None) == vsl.VSL_E_INVALID
    ok(vsl, H.vsl_gemm_f16(dev.p(A), dev.p(B), 64, 4096, 4096, dev.p(C), vsl.GEMM_A_F8 | vsl.GEMM_B8_SHIFT(-16), None))
    ok(vsl, H.vsl_gemm_f16(dev.p(A), dev.p(B), 64, 4096, 4096, dev.p(C), vsl.GEMM_A_F8 | vsl.GEMM_B8_SHIFT(30), None))


def test_gemm_f8lo_forms_refused(vsl, dev, H):
    A = dev.put(np.zeros((3 * 64 * 4096,), np.uint8))
    B = dev.put(np.zeros((4096, 4096), np.float16))
    C = dev.put(np.zeros((64, 4096), np.float32))
    # N a multiple of 128 (what every form needs) but not of the 256-wide tile; N not even that
    assert H.vsl_gemm_f16(dev.p(A), dev.p(B), 64, 3968, 4096, dev.p(C), vsl.GEMM_A_F8, None) == vsl.VSL_E_UNSUPPORTED
    assert H.vsl_gemm_f16(dev.p(A), dev.p(B), 64, 4000, 4096, dev.p(C), vsl.GEMM_A_F8, None) == vsl.VSL_E_INVALID
    # two A forms at once, an F8 output on a non-SwiGLU epilogue
    assert H.vsl_gemm_f16(dev.p(A), dev.p(B), 64, 4096, 4096, dev.p(C), vsl.GEMM_A_F8 | vsl.GEMM_A_X2,
                          None) == vsl.VSL_E_INVALID
    assert H.vsl_gemm_f16(dev.p(A), dev.p(B), 64, 4096, 4096, dev.p(C), vsl.GEMM_C_F8, None) == vsl.VSL_E_INVALID


@pytest.mark.parametrize("M,N,K", [(512, 4096, 14336), (300, 2048, 8192)])
def test_resid_rmsnorm_f8lo(vsl, orc, dev, H, M, N, K):
    """The down projection's entry with an F16F8 input and an F16F8 normalized output: the fused launch
    (K split) leaves x exactly as the unfused residual GEMM does, and both it and the unsplit path
    encode the oracle's RMSNorm of the updated rows."""
    rng = np.random.default_rng(M + N + K + 5)
    A = rng.normal(0, 1, (M, K)).astype(np.float32)
    B = rng.normal(0, 0.02, (N, K)).astype(np.float16)
    x0 = rng.normal(0, 1, (M, N)).astype(np.float32)
    g = rng.normal(1, 0.1, N).astype(np.float32)
    dA, hi, val = f8_buffer(dev, A)
    dB, dg = dev.put(B), dev.put(g)
    need = H.vsl_gemm_f16_ws_bytes(M, N, K, 2 | vsl.GEMM_A_F8)
    ws = dev.empty((need // 4 + 4,), np.float32)
    res = {}
    for mode in ("fused", "unfused", "unsplit"):
        x = dev.put(x0)
        xn = dev.empty((3 * M * N,), np.uint8)
        if mode == "unfused":
            ok(vsl, H.vsl_gemm_f16_ws(dev.p(dA), dev.p(dB), M, N, K, dev.p(x), 2 | vsl.GEMM_A_F8, dev.p(ws), need,
                                      None))
        else:
            ok(vsl, H.vsl_gemm_f16_resid_rmsnorm(dev.p(dA), dev.p(dB), M, N, K, vsl.GEMM_A_F8, dev.p(x), dev.p(dg),
                                                 1e-5, dev.p(xn), vsl.VSL_DT_F16F8,
                                                 dev.p(ws) if mode == "fused" else None,
                                                 need if mode == "fused" else 0, None))
        res[mode] = (dev.get(x).astype(np.float32), f8_read(dev, xn, M, N))
    assert np.array_equal(res["fused"][0], res["unfused"][0])
    rows = np.unique(np.concatenate([[0, M - 1], rng.integers(0, M, 24)]))
    ref = x0[rows].astype(np.float64) + T.f8lo_product(hi[rows], val[rows] - hi[rows].astype(np.float64), B)
    for mode in ("fused", "unsplit"):
        x, (hn, vn) = res[mode]
        assert rel_err(x[rows], ref) < 1e-5
        nref = np.stack([orc.rmsnorm(x[r], g, 1e-5) for r in rows]).astype(np.float64)
        assert_f8_encodes(hn[rows], vn[rows], nref)


@pytest.mark.parametrize("hd,nq,nkv,S,pos0", [(128, 8, 2, 300, 0), (64, 4, 4, 97, 37), (128, 32, 8, 512, 0),
                                              (128, 32, 8, 1024, 0)])
def test_attn_prefill_f16f8_output(vsl, dev, H, hd, nq, nkv, S, pos0):
    """The prefill attention writing its output as F16F8: the same hi plane as the hi/lo fp16 output of
    the same call, bit for bit, and hi + lo8 2^-12 within e4m3 precision of hi + lo (so every byte sits
    at its lo8_pos position)."""
    rng = np.random.default_rng(hd + nq + S + pos0)
    cap = 1024
    q = dev.put(rng.normal(0, 1, (2, S, nq * hd)).astype(np.float16) * np.array([1.0, 2.0 ** -11], np.float16)[:, None, None])
    kc = dev.put(rng.normal(0, 1, (nkv, cap, hd)).astype(np.float16))
    vc = dev.put(rng.normal(0, 1, (nkv, cap, hd)).astype(np.float16))
    scale = 1.0 / np.sqrt(hd)
    out2 = dev.empty((2, S, nq * hd), np.float16)
    ok(vsl, H.vsl_attn_prefill(dev.p(q), vsl.VSL_DT_F16X2, dev.p(kc), dev.p(vc), S, pos0, nq, nkv, hd, cap, scale,
                               dev.p(out2), vsl.VSL_DT_F16X2, None))
    out8 = dev.empty((3 * S * nq * hd,), np.uint8)
    ok(vsl, H.vsl_attn_prefill(dev.p(q), vsl.VSL_DT_F16X2, dev.p(kc), dev.p(vc), S, pos0, nq, nkv, hd, cap, scale,
                               dev.p(out8), vsl.VSL_DT_F16F8, None))
    o2 = dev.get(out2)
    hi8, val8 = f8_read(dev, out8, S, nq * hd)
    assert np.array_equal(hi8.view(np.uint16), o2[0].view(np.uint16))
    v2 = o2[0].astype(np.float64) + o2[1].astype(np.float64)
    assert np.all(np.abs(val8 - v2) <= F8_VALUE_REL * np.abs(v2) + F8_VALUE_ABS)
