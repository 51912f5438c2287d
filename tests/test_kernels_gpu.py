"""Kernel-level parity on the GPU: every op of include/vsl_hip.h against the oracle on the same
seeded inputs, called through the C ABI.  Device memory comes from torch (plumbing only)."""
import ctypes
import math

import numpy as np
import pytest

import vsl_testlib

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def _dev():
    return vsl_testlib.Dev()


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


# ------------------------------------------------------------------------------------------
# GEMV sweep (y = W X, fp16 W, fp32 accumulate)
# ------------------------------------------------------------------------------------------
SWEEP = [(4096, 4096), (14336, 4096), (4096, 14336), (32000, 4096)]


@pytest.mark.parametrize("N,K", SWEEP)
@pytest.mark.parametrize("B", [1, 4, 16])
def test_gemv_sweep(vsl, orc, dev, H, N, K, B):
    rng = np.random.default_rng(N * 131 + K * 7 + B)
    W = rng.normal(0, 0.02, (N, K)).astype(np.float16)
    X = rng.normal(0, 1, (K, B)).astype(np.float16)
    ref = orc.gemm_nt(W, X.astype(np.float32))
    dW = dev.put(W)
    if B == 1:  # the decode GEMV (fp32 activation)
        dX = dev.put(X.astype(np.float32))
        dY = dev.empty((N, 1), np.float32)
        ok(vsl, H.vsl_gemv(dev.p(dW), vsl.VSL_DT_F16, N, K, dev.p(dX), vsl.VSL_DT_F32, 1, dev.p(dY),
                           vsl.VSL_DT_F32, None))
        y = dev.get(dY)
        assert rel_err(y, ref) < 1e-5
    # the sweep as specified: fp16 X, fp16 Y
    dX = dev.put(X)
    dY = dev.empty((N, B), np.float16)
    ok(vsl, H.vsl_gemv(dev.p(dW), vsl.VSL_DT_F16, N, K, dev.p(dX), vsl.VSL_DT_F16, B, dev.p(dY),
                       vsl.VSL_DT_F16, None))
    y = dev.get(dY).astype(np.float32)
    # fp16 output: within half an fp16 ulp of the fp32-accumulated value, plus accumulation noise
    assert np.all(np.abs(y - ref) <= np.abs(ref) * 2.0 ** -11 + 1e-4 * np.max(np.abs(ref)))
    # fp32 output of the same product
    dY32 = dev.empty((N, B), np.float32)
    ok(vsl, H.vsl_gemv(dev.p(dW), vsl.VSL_DT_F16, N, K, dev.p(dX), vsl.VSL_DT_F16, B, dev.p(dY32),
                       vsl.VSL_DT_F32, None))
    assert rel_err(dev.get(dY32), ref) < 1e-5
    # batch of B contiguous activation vectors: X [B][K], Y [B][N]
    dXt = dev.put(np.ascontiguousarray(X.T))
    dYt = dev.empty((B, N), np.float32)
    ok(vsl, H.vsl_gemv_batched(dev.p(dW), N, K, dev.p(dXt), B, dev.p(dYt), vsl.VSL_DT_F32, None))
    assert rel_err(dev.get(dYt).T, ref) < 1e-5


@pytest.mark.parametrize("N,K,B", [(9000, 1536, 12), (8200, 512, 16), (16, 512, 1), (8193, 2560, 8), (8191, 1024, 9),
                                   (9000, 2048, 12), (8191, 4096, 9), (17, 6144, 16), (1, 3072, 13),
                                   (13000, 2048, 16), (26003, 1024, 11)])
def test_gemv_batched_ragged(vsl, orc, dev, H, N, K, B):
    """The sweep kernel on shapes outside the sweep: N not a multiple of the 16- or 32-row tiles (the
    two-tile blocks from N >= 8192 and B >= 8), K a multiple of 512 only, B neither 1, 4 nor 16;
    X [B][K] and X [K][B] layouts. With K % 1024 == 0 and B > 8 the [B][K] product stages both
    operands through LDS (a single row, 17 rows, vectors past B masked; 1536 and 2560 keep the
    register-fragment kernel), with two (N >= 12800) or four (N >= 25600) 16-row groups per block
    sharing each staged X chunk (13000 and 26003 rows: the last block partly past N)."""
    rng = np.random.default_rng(N + K + B)
    W = rng.normal(0, 0.02, (N, K)).astype(np.float16)
    X = rng.normal(0, 1, (K, B)).astype(np.float16)
    ref = orc.gemm_nt(W, X.astype(np.float32))
    dW = dev.put(W)
    dYt = dev.empty((B, N), np.float32)
    ok(vsl, H.vsl_gemv_batched(dev.p(dW), N, K, dev.p(dev.put(np.ascontiguousarray(X.T))), B, dev.p(dYt),
                               vsl.VSL_DT_F32, None))
    assert rel_err(dev.get(dYt).T, ref) < 1e-5
    dY = dev.empty((N, B), np.float32)
    ok(vsl, H.vsl_gemv(dev.p(dW), vsl.VSL_DT_F16, N, K, dev.p(dev.put(X)), vsl.VSL_DT_F16, B, dev.p(dY),
                       vsl.VSL_DT_F32, None))
    assert rel_err(dev.get(dY), ref) < 1e-5


@pytest.mark.parametrize("N,K,B,ydt", [(1, 1024, 2, 0), (37, 2048, 3, 0), (4099, 3072, 5, 0), (1000, 8192, 8, 0),
                                       (515, 1024, 7, 1), (3001, 4096, 4, 1), (4100, 6144, 6, 0), (300, 9216, 8, 0)])
def test_gemv_batched_rows(vsl, orc, dev, H, N, K, B, ydt):
    """The row-streaming kernel of the batched product (2 <= B <= 8, X [B][K] up to 128 KB in LDS,
    K % 1024 == 0): one row, odd row counts (a wave's second row past N), every B from 2 to 8, X at
    the 128 KB limit (B = 8, K = 8192); fp32 and fp16 Y.  B = 8 with K = 9216 is past the limit and
    takes the MFMA kernel."""
    rng = np.random.default_rng(N * 7 + K + B)
    W = rng.normal(0, 0.02, (N, K)).astype(np.float16)
    X = rng.normal(0, 1, (B, K)).astype(np.float16)
    ref = orc.gemm_nt(W, np.ascontiguousarray(X.T).astype(np.float32))  # [N][B]
    if ydt == 0:
        dY = dev.empty((B, N), np.float32)
        ok(vsl, H.vsl_gemv_batched(dev.p(dev.put(W)), N, K, dev.p(dev.put(X)), B, dev.p(dY), vsl.VSL_DT_F32, None))
        assert rel_err(dev.get(dY).T, ref) < 1e-5
    else:
        dY = dev.empty((B, N), np.float16)
        ok(vsl, H.vsl_gemv_batched(dev.p(dev.put(W)), N, K, dev.p(dev.put(X)), B, dev.p(dY), vsl.VSL_DT_F16, None))
        y = dev.get(dY).astype(np.float32).T
        assert np.all(np.abs(y - ref) <= np.abs(ref) * 2.0 ** -11 + 1e-4 * np.max(np.abs(ref)))


@pytest.mark.parametrize("B,off", [(1, 1), (1, 4), (4, 1), (12, 3)])
def test_gemv_batched_x_offset(vsl, orc, dev, H, B, off):
    """X starting `off` halfs past an aligned address: B = 1 takes the decode GEMV (8-byte X loads) only
    when X is 8-byte aligned, the other routes take X at any 2-byte alignment; the same result."""
    N, K = 2048, 4096
    rng = np.random.default_rng(B * 10 + off)
    W = rng.normal(0, 0.02, (N, K)).astype(np.float16)
    X = rng.normal(0, 1, (B, K)).astype(np.float16)
    ref = orc.gemm_nt(W, np.ascontiguousarray(X.T).astype(np.float32))
    buf = dev.put(np.concatenate([np.zeros(off, np.float16), X.reshape(-1), np.zeros(8, np.float16)]))
    dY = dev.empty((B, N), np.float32)
    ok(vsl, H.vsl_gemv_batched(dev.p(dev.put(W)), N, K, dev.p(buf) + 2 * off, B, dev.p(dY), vsl.VSL_DT_F32, None))
    assert rel_err(dev.get(dY).T, ref) < 1e-5


def test_gemv_rejects_bad_shapes(vsl, dev, H):
    d = dev.empty((16,), np.float32)
    assert H.vsl_gemv_batched(dev.p(d), 4, 1000, dev.p(d), 1, dev.p(d), 0, None) == -100  # K % 512
    assert H.vsl_gemv_batched(dev.p(d), 4, 2048, dev.p(d), 0, dev.p(d), 0, None) == -100  # B < 1
    assert H.vsl_gemv(dev.p(d), 1, 4, 12, dev.p(d), 0, 1, dev.p(d), 0, None) == -100  # K % 8
    assert H.vsl_gemv(dev.p(d), 1, 4, 16, dev.p(d), 0, 17, dev.p(d), 0, None) == -100  # B > 16
    assert H.vsl_gemv(None, 1, 4, 16, dev.p(d), 0, 1, dev.p(d), 0, None) == -100


# ------------------------------------------------------------------------------------------
# decode-step ops
# ------------------------------------------------------------------------------------------
def ctrl_buf(vsl, dev, H, pos, max_steps=4, cap=64, stop=0):
    c = dev.empty((8,), np.int32)
    ok(vsl, H.vsl_ctrl_reset(dev.p(c), pos, max_steps, stop, cap, None))
    return c


def rope_tables(cap, hd, theta):
    j = np.arange(hd // 2, dtype=np.float64)
    f = theta ** (-(2 * j) / hd)
    a = np.arange(cap, dtype=np.float64)[:, None] * f[None, :]
    return np.cos(a).astype(np.float32), np.sin(a).astype(np.float32)


@pytest.mark.parametrize("wdt,kvdt,d,nq,nkv,hd", [(1, 1, 4096, 32, 8, 128), (1, 1, 2048, 32, 8, 64),
                                                  (0, 0, 256, 4, 4, 64)])
def test_qkv_rope_append(vsl, orc, dev, H, wdt, kvdt, d, nq, nkv, hd):
    rng = np.random.default_rng(d + nq)
    cap, pos, theta, eps = 64, 37, 500000.0, 1e-5
    wnp = np.float16 if wdt == 1 else np.float32
    kvnp = np.float16 if kvdt == 1 else np.float32
    N = (nq + 2 * nkv) * hd
    W = rng.normal(0, 0.02, (N, d)).astype(wnp)
    x = rng.normal(0, 1, d).astype(np.float32)
    g = rng.normal(1, 0.1, d).astype(np.float32)
    cs, sn = rope_tables(cap, hd, theta)
    kc = dev.empty((nkv, cap, hd), kvnp)
    vc = dev.empty((nkv, cap, hd), kvnp)
    q = dev.empty((nq * hd,), np.float32)
    c = ctrl_buf(vsl, dev, H, pos, cap=cap)
    dcs, dsn = dev.put(cs), dev.put(sn)
    ok(vsl, H.vsl_qkv_rope_append(dev.p(dev.put(x)), dev.p(dev.put(g)), eps, dev.p(dev.put(W)), wdt, d, nq, nkv, hd,
                                  dev.p(dcs), dev.p(dsn), dev.p(kc), dev.p(vc), kvdt, cap, dev.p(q), dev.p(c), None))
    n = orc.rmsnorm(x, g, eps)
    y = orc.gemm_nt(W, n)[:, 0]
    qr = orc.rope(y[:nq * hd], nq, hd, pos, theta)
    kr = orc.rope(y[nq * hd:(nq + nkv) * hd], nkv, hd, pos, theta)
    vr = y[(nq + nkv) * hd:]
    tol = 1e-5 if wdt == 0 else 1e-4
    assert rel_err(dev.get(q), qr) < tol
    K = dev.get(kc).astype(np.float32)
    V = dev.get(vc).astype(np.float32)
    kt = 2.0 ** -10 if kvdt == 1 else tol
    assert rel_err(K[:, pos].reshape(-1), kr) < kt
    assert rel_err(V[:, pos].reshape(-1), vr) < kt
    assert np.all(K[:, :pos] == 0) and np.all(K[:, pos + 1:] == 0)  # only position `pos` is written


def test_qkv_capacity_guard(vsl, dev, H):
    """A position at or beyond the capacity makes the kernels refuse (error flag, done) instead of
    writing past the cache."""
    d, nq, nkv, hd, cap = 256, 4, 4, 64, 8
    c = ctrl_buf(vsl, dev, H, cap, cap=cap)
    W = dev.empty(((nq + 2 * nkv) * hd, d), np.float32)
    kc = dev.empty((nkv, cap, hd), np.float32)
    x = dev.empty((d,), np.float32)
    t = dev.empty((cap, hd // 2), np.float32)
    q = dev.empty((nq * hd,), np.float32)
    ok(vsl, H.vsl_qkv_rope_append(dev.p(x), None, 1e-5, dev.p(W), 0, d, nq, nkv, hd, dev.p(t), dev.p(t), dev.p(kc),
                                  dev.p(kc), 0, cap, dev.p(q), dev.p(c), None))
    ctrl = dev.get(c)
    assert ctrl[2] == 1 and ctrl[7] == 1


_LAYOUTS = [(1, 128, 32, 8), (1, 64, 32, 8), (0, 64, 4, 4), (1, 128, 8, 8)]
# GQA groups that are not powers of two: 3 (24/8 heads, the Llama-3.2-3B layout), 5, 6 and 7
_ODD_GQA = [(1, 128, 24, 8), (0, 64, 15, 3), (1, 64, 12, 2), (1, 128, 14, 2)]
_LENGTHS = [1, 5, 300, 1025]
# every head layout at the engine's 32 splits; the split sweep on two layouts
_ATTN_CASES = ([(lay, n, 32) for lay in _LAYOUTS + _ODD_GQA for n in _LENGTHS] +
               [(lay, n, s) for lay in ((1, 128, 32, 8), (0, 64, 4, 4)) for n in _LENGTHS for s in (1, 7, 48, 100)] +
               [(lay, n, 7) for lay in _ODD_GQA for n in (5, 1025)])


def _nan_past(cache, length):
    """Cache rows at and past the attended length hold NaN: they are never written before they are
    read by a later step, so the kernels must not let them reach the output."""
    cache[:, length:] = np.nan
    return cache


@pytest.mark.parametrize("layout,length,nsplit", _ATTN_CASES)
def test_attn_decode(vsl, orc, dev, H, layout, length, nsplit):
    """Split-KV decode attention against the oracle: split counts 1 (a single block walks every
    tile), 7 (ragged tile ownership), 32 (the engine's default), 48 (the combine's 64-split register
    path) and 100 (more than the combine's register paths hold); cache rows past the length are NaN."""
    kvdt, hd, nq, nkv = layout
    rng = np.random.default_rng(length * 3 + hd)
    cap = 2048
    kvnp = np.float16 if kvdt == 1 else np.float32
    K = _nan_past(rng.normal(0, 1, (nkv, cap, hd)).astype(kvnp), length)
    V = _nan_past(rng.normal(0, 1, (nkv, cap, hd)).astype(kvnp), length)
    q = rng.normal(0, 1, nq * hd).astype(np.float32)
    scale = 1.0 / math.sqrt(hd)
    po = dev.empty((nq * nsplit * hd,), np.float32)
    pml = dev.empty((nq * nsplit * 2,), np.float32)
    out = dev.empty((nq * hd,), np.float32)
    c = ctrl_buf(vsl, dev, H, length - 1, cap=cap)
    ok(vsl, H.vsl_attn_decode(dev.p(dev.put(q)), dev.p(dev.put(K)), dev.p(dev.put(V)), kvdt, nq, nkv, hd, cap, scale,
                              nsplit, dev.p(po), dev.p(pml), dev.p(out), dev.p(c), None))
    ref = orc.attention_decode(q, K.astype(np.float32), V.astype(np.float32), nq, nkv, hd, cap, length, scale)
    got = dev.get(out)
    assert np.all(np.isfinite(got))
    assert rel_err(got, ref) < 2e-5


_LONG_LENGTHS = [1, 5, 17, 300, 1025, 9000, 16384]
# GQA groups of 4, 1, 2 and 8 heads at 32 splits; the split sweep on the 8B layout (one block over
# the whole 16384-position cache is left to the 9000-position case)
_LONG_CASES = ([(nq, n, 32) for nq in (32, 8, 16, 64) for n in _LONG_LENGTHS] +
               [(32, n, s) for s in (1, 7, 100) for n in _LONG_LENGTHS if not (n == 16384 and s == 1)] +
               [(nq, n, 32) for nq in (24, 40, 48, 56) for n in (5, 9000, 16384)])


@pytest.mark.parametrize("nq,length,nsplit", _LONG_CASES)
def test_attn_decode_long_cache(vsl, orc, dev, H, nq, length, nsplit):
    """fp16 caches of head_dim 128 above 8192 positions of capacity run the matrix-core kernel (scores
    from hi + lo fp16 planes of q on MFMA, 16-position tiles per wave): against the oracle for GQA
    groups of 4, 1, 2, 8, 3, 5, 6 and 7 heads, lengths from one position to the full cache, the split counts of
    the short-cache test; cache rows past the length are NaN (the kernel requests its first two tiles
    before it knows the length)."""
    nkv, hd, cap = 8, 128, 16384
    rng = np.random.default_rng(length * 7 + nq + nsplit)
    K = _nan_past(rng.normal(0, 1, (nkv, cap, hd)).astype(np.float16), length)
    V = _nan_past(rng.normal(0, 1, (nkv, cap, hd)).astype(np.float16), length)
    q = rng.normal(0, 1, nq * hd).astype(np.float32)
    scale = 1.0 / math.sqrt(hd)
    po = dev.empty((nq * nsplit * hd,), np.float32)
    pml = dev.empty((nq * nsplit * 2,), np.float32)
    out = dev.empty((nq * hd,), np.float32)
    c = ctrl_buf(vsl, dev, H, length - 1, cap=cap)
    ok(vsl, H.vsl_attn_decode(dev.p(dev.put(q)), dev.p(dev.put(K)), dev.p(dev.put(V)), 1, nq, nkv, hd, cap, scale,
                              nsplit, dev.p(po), dev.p(pml), dev.p(out), dev.p(c), None))
    ref = orc.attention_decode(q, K.astype(np.float32), V.astype(np.float32), nq, nkv, hd, cap, length, scale)
    got = dev.get(out)
    assert np.all(np.isfinite(got))
    assert rel_err(got, ref) < 2e-5


@pytest.mark.parametrize("kvdt,hd,nq,nkv", [(1, 128, 32, 8), (0, 64, 4, 4), (1, 128, 24, 8)])
@pytest.mark.parametrize("length,window,n_glob,thr", [
    (300, 64, 4, 100),    # windowed: globals 0..3 and keys 235..299
    (300, 64, 4, 300),    # threshold not passed: dense
    (1025, 100, 16, 0),   # windowed from the start; 16 globals span a whole tile
    (70, 64, 4, 0),       # window and globals leave out key 4 only
    (69, 64, 4, 0),       # window and globals cover every key: dense
    (2000, 512, 16, 8),   # the reference's window and globals
])
@pytest.mark.parametrize("nsplit", [32, 7])
def test_attn_decode_window(vsl, orc, dev, H, kvdt, hd, nq, nkv, length, window, n_glob, thr, nsplit):
    """Windowed decode attention (virtual positions remapped past the globals) against the oracle's
    windowed attention; keys outside the window are filled with large values that would dominate."""
    rng = np.random.default_rng(length + window + hd)
    cap = 2048
    kvnp = np.float16 if kvdt == 1 else np.float32
    K = rng.normal(0, 1, (nkv, cap, hd)).astype(np.float32)
    V = rng.normal(0, 1, (nkv, cap, hd)).astype(np.float32)
    q = rng.normal(0, 1, nq * hd).astype(np.float32)
    p = length - 1
    if length > thr and p > n_glob + window:
        hidden = slice(n_glob, p - window)
        K[:, hidden] = np.repeat(q.reshape(nq, hd)[::nq // nkv][:, None, :], p - window - n_glob, axis=1) * 4
        V[:, hidden] = 100.0
    K, V = _nan_past(K, length).astype(kvnp), _nan_past(V, length).astype(kvnp)
    scale = 1.0 / math.sqrt(hd)
    po = dev.empty((nq * nsplit * hd,), np.float32)
    pml = dev.empty((nq * nsplit * 2,), np.float32)
    out = dev.empty((nq * hd,), np.float32)
    c = ctrl_buf(vsl, dev, H, p, cap=cap)
    ok(vsl, H.vsl_attn_decode_window(dev.p(dev.put(q)), dev.p(dev.put(K)), dev.p(dev.put(V)), kvdt, nq, nkv, hd,
                                     cap, scale, nsplit, dev.p(po), dev.p(pml), dev.p(out), dev.p(c), window, n_glob,
                                     thr, None))
    ref = orc.attention_decode(q, K.astype(np.float32), V.astype(np.float32), nq, nkv, hd, cap, length, scale,
                               window=(window, n_glob, thr))
    assert rel_err(dev.get(out), ref) < 2e-5


@pytest.mark.parametrize("hd,nq,nkv,S,pos0,window,n_glob,thr,x2", [
    (64, 8, 8, 300, 100, 64, 4, 150, False),      # rows 100..149 dense, 150..399 windowed, tiles skipped
    (128, 32, 8, 200, 0, 100, 70, 60, False),     # globals over two tiles; a block straddles the threshold
    (128, 32, 8, 160, 300, 32, 0, 0, True),       # every row windowed, no globals, split q / out
    (64, 8, 8, 96, 0, 512, 16, 8192, False),      # threshold not reached: dense
    (128, 32, 8, 192, 1000, 512, 16, 900, True),  # every row windowed, tiles wholly inside every window
    (64, 8, 8, 160, 700, 256, 128, 600, False),   # two whole global tiles, then the windows
    (128, 24, 8, 200, 0, 100, 70, 60, True),      # GQA 3 (one head per block), split q / out
    (64, 12, 2, 160, 300, 32, 0, 0, False),       # GQA 6 (two heads per block), every row windowed
])
def test_attn_prefill_window(vsl, orc, dev, H, hd, nq, nkv, S, pos0, window, n_glob, thr, x2):
    rng = np.random.default_rng(hd + S + pos0 + window)
    cap = max(512, -(-(pos0 + S) // 512) * 512)
    Q = rng.normal(0, 1, (S, nq * hd)).astype(np.float32)
    K = rng.normal(0, 1, (nkv, cap, hd)).astype(np.float16)
    V = rng.normal(0, 1, (nkv, cap, hd)).astype(np.float16)
    if x2:
        hi = Q.astype(np.float16)
        lo = (Q - hi.astype(np.float32)).astype(np.float16)
        qd, qdt, odt = np.concatenate([hi, lo]), 2, 2
    else:
        qd, qdt, odt = Q.astype(np.float16), 1, 1
        Q = qd.astype(np.float32)
    out = dev.empty(((2 if x2 else 1) * S, nq * hd), np.float16)
    scale = 1.0 / math.sqrt(hd)
    ok(vsl, H.vsl_attn_prefill_window(dev.p(dev.put(qd)), qdt, dev.p(dev.put(K)), dev.p(dev.put(V)), S, pos0, nq,
                                      nkv, hd, cap, scale, dev.p(out), odt, window, n_glob, thr, None))
    O = dev.get(out).astype(np.float32)
    if x2:
        O = O[:S] + O[S:]
    Kf, Vf = K.astype(np.float32), V.astype(np.float32)
    for s in sorted(set(list(range(0, S, max(1, S // 11))) + [S - 1, min(S - 1, max(0, thr - pos0 - 1)),
                                                             min(S - 1, max(0, thr - pos0))])):
        ref = orc.attention_decode(Q[s], Kf, Vf, nq, nkv, hd, cap, pos0 + s + 1, scale, window=(window, n_glob, thr))
        assert rel_err(O[s], ref) < (1e-4 if x2 else 4e-3), s


def test_gemv_residual_and_swiglu(vsl, orc, dev, H):
    rng = np.random.default_rng(9)
    d, F = 4096, 14336
    Wd = rng.normal(0, 0.02, (d, F)).astype(np.float16)
    h = rng.normal(0, 1, F).astype(np.float32)
    r = rng.normal(0, 1, d).astype(np.float32)
    dr = dev.put(r)
    ok(vsl, H.vsl_gemv_residual(dev.p(dev.put(Wd)), 1, d, F, dev.p(dev.put(h)), dev.p(dr), None, None))
    assert rel_err(dev.get(dr), r + orc.gemm_nt(Wd, h)[:, 0]) < 1e-5
    Wgu = rng.normal(0, 0.02, (2 * F, d)).astype(np.float16)
    x = rng.normal(0, 1, d).astype(np.float32)
    gm = rng.normal(1, 0.1, d).astype(np.float32)
    dh = dev.empty((F,), np.float32)
    ok(vsl, H.vsl_norm_swiglu(dev.p(dev.put(x)), dev.p(dev.put(gm)), 1e-5, dev.p(dev.put(Wgu)), 1, d, F, dev.p(dh),
                              None, None))
    m = orc.rmsnorm(x, gm, 1e-5)
    gu = orc.gemm_nt(Wgu, m)[:, 0]
    assert rel_err(dev.get(dh), orc.swiglu(gu[:F], gu[F:])) < 1e-4


@pytest.mark.parametrize("N,K", [(77, 8), (300, 40), (1000, 1000), (4099, 4104), (129, 8200), (64, 14344),
                                 (20, 16392)])
def test_gemv_ragged_k(vsl, orc, dev, H, N, K):
    """Decode GEMVs whose K is a multiple of 8 but not of 32: the staged activation vector's last
    aligned group of eight float4 slots is partial (4-, 8- and 16-wave blocks). Residual GEMV, fp32-X
    GEMV and RMSNorm + SwiGLU against the oracle."""
    rng = np.random.default_rng(3 * N + K)
    W = rng.normal(0, 0.02, (N, K)).astype(np.float16)
    h = rng.normal(0, 1, K).astype(np.float32)
    r = rng.normal(0, 1, N).astype(np.float32)
    dW, dr = dev.put(W), dev.put(r)
    ref = orc.gemm_nt(W, h)[:, 0]
    ok(vsl, H.vsl_gemv_residual(dev.p(dW), 1, N, K, dev.p(dev.put(h)), dev.p(dr), None, None))
    assert rel_err(dev.get(dr), r + ref) < 1e-5
    dy = dev.empty((N,), np.float32)
    ok(vsl, H.vsl_gemv(dev.p(dW), vsl.VSL_DT_F16, N, K, dev.p(dev.put(h)), vsl.VSL_DT_F32, 1, dev.p(dy),
                       vsl.VSL_DT_F32, None))
    assert rel_err(dev.get(dy), ref) < 1e-5
    F = N // 2
    if F:
        gm = rng.normal(1, 0.1, K).astype(np.float32)
        dh = dev.empty((F,), np.float32)
        ok(vsl, H.vsl_norm_swiglu(dev.p(dev.put(h)), dev.p(dev.put(gm)), 1e-5, dev.p(dW), 1, K, F, dev.p(dh),
                                  None, None))
        gu = orc.gemm_nt(W[:2 * F], orc.rmsnorm(h, gm, 1e-5))[:, 0]
        assert rel_err(dev.get(dh), orc.swiglu(gu[:F], gu[F:])) < 1e-4


@pytest.mark.parametrize("N,K", [(4100, 28672), (1000, 20480), (333, 32768)])
def test_gemv_wide_k(vsl, orc, dev, H, N, K):
    """Decode GEMVs wider than 16384 columns (70B-class down projections: K = 28672) stage the fp32
    activation in up to 128 KB of LDS with one 16-wave block per CU: the residual GEMV, the fp32-X and
    the fp16-X GEMV against the oracle, and K past 32768 refused."""
    rng = np.random.default_rng(N + K)
    W = rng.normal(0, 0.02, (N, K)).astype(np.float16)
    h = rng.normal(0, 1, K).astype(np.float32)
    r = rng.normal(0, 1, N).astype(np.float32)
    dW, dr = dev.put(W), dev.put(r)
    ref = orc.gemm_nt(W, h)[:, 0]
    ok(vsl, H.vsl_gemv_residual(dev.p(dW), 1, N, K, dev.p(dev.put(h)), dev.p(dr), None, None))
    assert rel_err(dev.get(dr), r + ref) < 1e-5
    dy = dev.empty((N,), np.float32)
    ok(vsl, H.vsl_gemv(dev.p(dW), vsl.VSL_DT_F16, N, K, dev.p(dev.put(h)), vsl.VSL_DT_F32, 1, dev.p(dy),
                       vsl.VSL_DT_F32, None))
    assert rel_err(dev.get(dy), ref) < 1e-5
    h16 = h.astype(np.float16)
    ok(vsl, H.vsl_gemv(dev.p(dW), vsl.VSL_DT_F16, N, K, dev.p(dev.put(h16)), vsl.VSL_DT_F16, 1, dev.p(dy),
                       vsl.VSL_DT_F32, None))
    assert rel_err(dev.get(dy), orc.gemm_nt(W, h16.astype(np.float32))[:, 0]) < 1e-5
    assert H.vsl_gemv_residual(dev.p(dW), 1, 8, 32776, dev.p(dW), dev.p(dr), None, None) == vsl.VSL_E_INVALID


def test_norm_swiglu_wide_k(vsl, orc, dev, H):
    """The RMSNorm + [Wgate; Wup] + SwiGLU GEMV past 16384 input columns (16-wave blocks, the norm
    over the staged vector) against the oracle."""
    rng = np.random.default_rng(77)
    d, F = 18432, 600
    Wgu = rng.normal(0, 0.02, (2 * F, d)).astype(np.float16)
    x = rng.normal(0, 1, d).astype(np.float32)
    gm = rng.normal(1, 0.1, d).astype(np.float32)
    dh = dev.empty((F,), np.float32)
    ok(vsl, H.vsl_norm_swiglu(dev.p(dev.put(x)), dev.p(dev.put(gm)), 1e-5, dev.p(dev.put(Wgu)), 1, d, F, dev.p(dh),
                              None, None))
    gu = orc.gemm_nt(Wgu, orc.rmsnorm(x, gm, 1e-5))[:, 0]
    assert rel_err(dev.get(dh), orc.swiglu(gu[:F], gu[F:])) < 1e-4


def test_lm_head_greedy_and_bookkeeping(vsl, orc, dev, H):
    rng = np.random.default_rng(12)
    V, d = 32000, 4096
    W = rng.normal(0, 0.02, (V, d)).astype(np.float16)
    E = rng.normal(0, 0.02, (V, d)).astype(np.float16)
    x = rng.normal(0, 1, d).astype(np.float32)
    g = np.ones(d, np.float32)
    nb = H.vsl_lm_head_ws_blocks()
    ws_v, ws_i = dev.empty((nb,), np.float32), dev.empty((nb,), np.int32)
    toks = dev.empty((8,), np.int32)
    logits = dev.empty((V,), np.float32)
    dx = dev.put(x)
    c = ctrl_buf(vsl, dev, H, 10, max_steps=2, cap=64)
    s = vsl.Sampler(0, 0.0, 40, 0, 0)
    ok(vsl, H.vsl_lm_head_sample(dev.p(dev.put(g)), 1e-5, dev.p(dev.put(W)), 1, V, d, dev.p(dx), dev.p(dev.put(E)), 1,
                                 dev.p(logits), s, dev.p(ws_v), dev.p(ws_i), dev.p(toks), dev.p(c), None))
    ref = orc.gemm_nt(W, orc.rmsnorm(x, g, 1e-5))[:, 0]
    lg = dev.get(logits)
    assert rel_err(lg, ref) < 1e-5
    t = int(dev.get(toks)[0])
    assert t == int(np.argmax(lg))
    srt = np.sort(ref)
    if srt[-1] - srt[-2] > 1e-3:
        assert t == int(np.argmax(ref))
    ctrl = dev.get(c)
    assert (ctrl[0], ctrl[1], ctrl[2], ctrl[5]) == (11, 1, 0, t)
    assert np.array_equal(dev.get(dx), E[t].astype(np.float32))  # next step's embedding row


def test_sample_logits_greedy_ties_and_topk(vsl, orc, dev, H):
    out = dev.empty((1,), np.int32)
    lg = np.zeros(32000, np.float32)
    lg[[77, 5000, 31999]] = 3.0
    ok(vsl, H.vsl_sample_logits(dev.p(dev.put(lg)), 32000, vsl.Sampler(0, 0.0, 40, 0, 0), 0, dev.p(out), None))
    assert dev.get(out)[0] == 77
    rng = np.random.default_rng(13)
    l = rng.normal(0, 1.3, 32000).astype(np.float32)
    dl = dev.put(l)
    for step in range(64):
        ok(vsl, H.vsl_sample_logits(dev.p(dl), 32000, vsl.Sampler(2, 0.7, 40, 0, 99), step, dev.p(out), None))
        assert dev.get(out)[0] == orc.sample(l, orc.SAMPLE_TOPK_SEEDED, 0.7, 40, 99, step)


def test_sample_logits_topk_limits(vsl, orc, dev, H):
    """Seeded top-k at the largest k of the one-wave path (64), the first k of the radix-select path
    (65), the largest single chunk (1024), the first two-chunk k (1025), k = V and top_k above V (all
    of V: 32 chunks, the walk gathering each again) against the oracle; k = 0 (which the oracle would
    read as all of V) and min(top_k, V) above VSL_MAX_TOP_K are refused with VSL_E_UNSUPPORTED by
    vsl_sample_logits and by vsl_lm_head_sample before anything is launched, and k = VSL_MAX_TOP_K
    (256 chunks) is served; top_k above a small V means all of V; every mode serves a 128256-entry
    vocabulary."""
    out = dev.empty((1,), np.int32)
    l = np.random.default_rng(21).normal(0, 1.0, 32000).astype(np.float32)
    dl = dev.put(l)
    for k in (64, 65, 1024, 1025, 32000, 0xFFFFFFFF):
        for step in range(16 if k <= 1025 else 6):
            ok(vsl, H.vsl_sample_logits(dev.p(dl), 32000, vsl.Sampler(2, 1.5, k, 0, 5), step, dev.p(out), None))
            assert dev.get(out)[0] == orc.sample(l, orc.SAMPLE_TOPK_SEEDED, 1.5, k, 5, step), (k, step)
    assert H.vsl_sample_logits(dev.p(dl), 32000, vsl.Sampler(2, 0.7, 0, 0, 5), 0, dev.p(out), None) == -103
    kmax = vsl.MAX_TOP_K
    huge = np.random.default_rng(24).normal(0, 1.0, kmax + 4000).astype(np.float32)
    dh = dev.put(huge)
    for k in (kmax + 1, 0xFFFFFFFF):
        assert H.vsl_sample_logits(dev.p(dh), huge.size, vsl.Sampler(2, 0.7, k, 0, 5), 0, dev.p(out), None) == -103
    for step in range(2):
        ok(vsl, H.vsl_sample_logits(dev.p(dh), huge.size, vsl.Sampler(2, 4.0, kmax, 0, 5), step, dev.p(out), None))
        assert dev.get(out)[0] == orc.sample(huge, orc.SAMPLE_TOPK_SEEDED, 4.0, kmax, 5, step), step
    big = np.random.default_rng(23).normal(0, 2.0, 128256).astype(np.float32)
    dbig = dev.put(big)
    for mode, T in ((0, 0.0), (1, 0.7), (2, 0.7)):
        for step in range(4):
            ok(vsl, H.vsl_sample_logits(dev.p(dbig), big.size, vsl.Sampler(mode, T, 40, 0, 5), step, dev.p(out), None))
            assert dev.get(out)[0] == orc.sample(big, mode, T, 40, 5, step), (mode, step)
    small = np.random.default_rng(22).normal(0, 1.0, 40).astype(np.float32)
    for step in range(8):
        ok(vsl, H.vsl_sample_logits(dev.p(dev.put(small)), 40, vsl.Sampler(2, 0.9, 50, 0, 6), step, dev.p(out), None))
        assert dev.get(out)[0] == orc.sample(small, orc.SAMPLE_TOPK_SEEDED, 0.9, 50, 6, step)
    V, d = 4096, 256
    nb = H.vsl_lm_head_ws_blocks()
    ws_v, ws_i = dev.empty((nb,), np.float32), dev.empty((nb,), np.int32)
    toks, logits = dev.empty((8,), np.int32), dev.empty((V,), np.float32)
    W = dev.empty((V, d), np.float16)
    x = dev.empty((d,), np.float32)
    c = ctrl_buf(vsl, dev, H, 3, max_steps=4, cap=64)
    before = dev.get(c).copy()
    rc = H.vsl_lm_head_sample(None, 1e-5, dev.p(W), 1, V, d, dev.p(x), dev.p(W), 1, dev.p(logits),
                              vsl.Sampler(2, 0.7, 0, 0, 1), dev.p(ws_v), dev.p(ws_i), dev.p(toks), dev.p(c), None)
    assert rc == -103
    assert np.array_equal(dev.get(c), before)  # nothing ran


def _topk_cases():
    """Logit vectors that take each selection route of the seeded top-k kernel: few elements above
    the threshold (normal logits), ties everywhere (all equal, small integers, +0 and -0), mostly
    -inf, a small V, and large values packed into 30 of the 1024 threads' index classes so that more
    than 1024 elements pass the threshold."""
    rng = np.random.default_rng(31)
    cases = {"normal": rng.normal(0, 1.3, 32000), "equal": np.zeros(32000),
             "integers": rng.integers(0, 3, 32000), "small": rng.normal(0, 1.0, 37)}
    z = rng.normal(0, 1.0, 5000)
    z[::3] = -0.0
    z[1::3] = 0.0
    cases["signed_zero"] = z
    inf = np.full(32000, -np.inf)
    inf[[5, 700, 20000, 31999]] = [1.0, 2.0, 2.0, 0.5]
    cases["mostly_neg_inf"] = inf
    packed = rng.normal(0, 1.0, 65536)
    packed[np.arange(65536) % 1024 < 30] += 50.0
    cases["packed_classes"] = packed
    return {n: v.astype(np.float32) for n, v in cases.items()}


@pytest.mark.parametrize("name", list(_topk_cases()))
def test_sample_topk_selection_routes(vsl, orc, dev, H, name):
    """Seeded top-k against the oracle on every selection route: k in {1, 40, 64} (the threshold from
    per-thread maxima), {65, 300, 1024} (the radix select, whose index passes the tied cases need) and
    {1025, 3000} (chunks of 1024 below each other's boundary key, the walk gathering them again)."""
    l = _topk_cases()[name]
    out = dev.empty((1,), np.int32)
    dl = dev.put(l)
    for k in (1, 40, 64, 65, 300, 1024, 1025, 3000):
        for step in range(6):
            ok(vsl, H.vsl_sample_logits(dev.p(dl), l.size, vsl.Sampler(2, 0.8, k, 0, 3), step, dev.p(out), None))
            assert dev.get(out)[0] == orc.sample(l, orc.SAMPLE_TOPK_SEEDED, 0.8, k, 3, step), (name, k, step)


def test_sample_topk_nan_logits(vsl, orc, dev, H):
    """NaN logits (where the reference's comparator has no order) rank below every number, lower
    index first.  With at least k numbers the draw equals the oracle's on the vector with the NaNs
    replaced by -inf (same k candidates, same weights); with fewer, a NaN weight reaches the sum and
    the walk returns the first candidate."""
    out = dev.empty((1,), np.int32)
    l = np.random.default_rng(51).normal(0, 1.0, 32000).astype(np.float32)
    l[::2] = np.nan
    masked = np.where(np.isnan(l), -np.inf, l).astype(np.float32)
    for k in (40, 500):
        for step in range(8):
            ok(vsl, H.vsl_sample_logits(dev.p(dev.put(l)), l.size, vsl.Sampler(2, 0.7, k, 0, 8), step, dev.p(out), None))
            assert dev.get(out)[0] == orc.sample(masked, orc.SAMPLE_TOPK_SEEDED, 0.7, k, 8, step)
    few = np.full(5000, np.nan, np.float32)
    few[[9, 3]] = [1.0, 1.0]
    for k in (40, 500):
        for step in range(4):
            ok(vsl, H.vsl_sample_logits(dev.p(dev.put(few)), few.size, vsl.Sampler(2, 0.7, k, 0, 8), step, dev.p(out),
                                        None))
            assert dev.get(out)[0] == 3


def test_sample_greedy_any_vocabulary(vsl, orc, dev, H):
    """Greedy over V above 65536 scans every logit; a NaN first logit gives token 0 (greedy_sampling
    starts from logits[0] and a NaN is never beaten), other NaNs never win."""
    out = dev.empty((1,), np.int32)
    l = np.random.default_rng(41).normal(0, 1.0, 70000).astype(np.float32)
    l[69000] = 9.0
    ok(vsl, H.vsl_sample_logits(dev.p(dev.put(l)), 70000, vsl.Sampler(0, 0.0, 40, 0, 0), 0, dev.p(out), None))
    assert dev.get(out)[0] == 69000 == orc.sample(l, orc.SAMPLE_GREEDY)
    l[123] = np.nan
    ok(vsl, H.vsl_sample_logits(dev.p(dev.put(l)), 70000, vsl.Sampler(2, 0.0, 40, 0, 0), 0, dev.p(out), None))
    assert dev.get(out)[0] == 69000 == orc.sample(l, orc.SAMPLE_GREEDY)
    l[0] = np.nan
    ok(vsl, H.vsl_sample_logits(dev.p(dev.put(l)), 70000, vsl.Sampler(0, 0.0, 40, 0, 0), 0, dev.p(out), None))
    assert dev.get(out)[0] == 0 == orc.sample(l, orc.SAMPLE_GREEDY)


def test_sample_reference_mode_is_softmax_argmax(vsl, orc, dev, H):
    """VSL_SAMPLE_REFERENCE restates the member top_k_sampling's tokens[0]: the first index of the
    largest fp32 probability exp(l/T - max)/sum.  Where logits next to the maximum differ by less than
    exp can resolve (here by ~1e-12 at 1e-6), their probabilities are equal and the lower index wins --
    the logit argmax would pick the larger logit.  On ordinary logits it is the argmax.  Both against
    the oracle's restatement; any NaN logit gives token 0 as in the reference's scan."""
    out = dev.empty((1,), np.int32)
    lg = np.full(32000, -5.0, np.float32)
    top = np.float32(1e-6)
    lg[3000] = top
    lg[1200] = np.nextafter(np.nextafter(top, np.float32(0)), np.float32(0))  # two ulps below, lower index
    for T in (0.7, 1.0, 1.3):
        r = orc.sample(lg, orc.SAMPLE_REFERENCE, T)
        assert r == 1200 and orc.sample(lg, orc.SAMPLE_GREEDY) == 3000
        ok(vsl, H.vsl_sample_logits(dev.p(dev.put(lg)), 32000, vsl.Sampler(1, T, 40, 0, 0), 0, dev.p(out), None))
        assert dev.get(out)[0] == r
    ok(vsl, H.vsl_sample_logits(dev.p(dev.put(lg)), 32000, vsl.Sampler(0, 0.0, 40, 0, 0), 0, dev.p(out), None))
    assert dev.get(out)[0] == 3000
    rng = np.random.default_rng(23)
    for i in range(8):
        l = rng.normal(0, 2.0, 32000).astype(np.float32)
        ok(vsl, H.vsl_sample_logits(dev.p(dev.put(l)), 32000, vsl.Sampler(1, 0.7, 40, 0, 0), 0, dev.p(out), None))
        assert dev.get(out)[0] == orc.sample(l, orc.SAMPLE_REFERENCE, 0.7) == int(np.argmax(l))
    l[17] = np.nan
    ok(vsl, H.vsl_sample_logits(dev.p(dev.put(l)), 32000, vsl.Sampler(1, 0.7, 40, 0, 0), 0, dev.p(out), None))
    assert dev.get(out)[0] == orc.sample(l, orc.SAMPLE_REFERENCE, 0.7) == 0


def test_embed_clamps_out_of_range_ids(vsl, dev, H):
    """embedding_lookup.comp:32: an id at or past the vocabulary reads row V - 1 (fp16 and fp32 tables)."""
    V, d = 300, 64
    for dt, npdt in ((1, np.float16), (0, np.float32)):
        E = np.random.default_rng(24).normal(0, 1, (V, d)).astype(npdt)
        ids = np.array([0, 5, V - 1, V, V + 7, 2**32 - 1], np.uint32)
        o = dev.empty((len(ids), d), np.float32)
        ok(vsl, H.vsl_embed(dev.p(dev.put(E)), dt, V, d, dev.p(dev.put(ids.view(np.int32))), len(ids), dev.p(o), None))
        want = E[np.minimum(ids, V - 1)].astype(np.float32)
        assert np.array_equal(dev.get(o), want)


# ------------------------------------------------------------------------------------------
# prefill ops
# ------------------------------------------------------------------------------------------
@pytest.mark.parametrize("M,N,K", [(1, 128, 32), (77, 256, 4096), (512, 6144, 4096), (200, 4096, 14336)])
@pytest.mark.parametrize("epi", [0, 1, 2])
def test_gemm_f16(vsl, dev, H, M, N, K, epi):
    rng = np.random.default_rng(M + N + K + epi)
    A = rng.normal(0, 1, (M, K)).astype(np.float16)
    B = rng.normal(0, 0.02, (N, K)).astype(np.float16)
    ref = A.astype(np.float64) @ B.astype(np.float64).T
    if epi == 1:
        C = dev.empty((M, N), np.float16)
    else:
        C0 = rng.normal(0, 1, (M, N)).astype(np.float32) if epi == 2 else np.zeros((M, N), np.float32)
        C = dev.put(C0)
        ref = ref + C0
    ok(vsl, H.vsl_gemm_f16(dev.p(dev.put(A)), dev.p(dev.put(B)), M, N, K, dev.p(C), epi, None))
    y = dev.get(C).astype(np.float64)
    tol = 2.0 ** -10 if epi == 1 else 1e-5
    assert rel_err(y, ref) < tol


@pytest.mark.parametrize("M,N,K,epi,ax2,cx2", [
    (512, 14336, 2048, 3, False, False),   # SwiGLU over [Wgate; Wup]: 2 x 112 tiles of 256 x 256
    (512, 14336, 2048, 3, True, True),     # split A (hi/lo planes) and split output
    (777, 14336, 1024, 3, True, False),    # ragged M
    (2048, 6144, 4096, 0, False, False),   # fp32 store
    (2048, 6144, 4096, 0, True, False),
    (1024, 12288, 128, 2, False, False),   # residual add; four K stages (one pass over the buffers)
    (1536, 8192, 256, 1, True, False),     # fp16 store; split A, four stages
    (2048, 4096, 1024, 2, True, False),    # 128 x 256 tiles (16 x 16 of them), split A
    (1536, 4096, 512, 3, False, True),     # 128 x 256 tiles, SwiGLU with split output
])
def test_gemm_dma(vsl, orc, dev, H, M, N, K, epi, ax2, cx2):
    """Shapes whose 256 x 256 (or 128 x 256) tiles cover >= 192 CUs run the direct-to-LDS GEMM:
    sampled rows (the first, the last, and random ones) against a float64 product."""
    rng = np.random.default_rng(M + N + K + epi + 7 * ax2)
    nb = 2 * N if epi == 3 else N
    Af = rng.normal(0, 1, (M, K)).astype(np.float32)
    B = rng.normal(0, 0.02, (nb, K)).astype(np.float16)
    if ax2:
        hi = Af.astype(np.float16)
        lo = (Af - hi.astype(np.float32)).astype(np.float16)
        Ad = np.concatenate([hi, lo])
        Aref = hi.astype(np.float64) + lo.astype(np.float64)
    else:
        Ad = Af.astype(np.float16)
        Aref = Ad.astype(np.float64)
    if epi == 1:
        C = dev.empty((M, N), np.float16)
    elif epi == 3:
        C = dev.empty(((2 if cx2 else 1) * M, N), np.float16)
    else:
        C0 = rng.normal(0, 1, (M, N)).astype(np.float32) if epi == 2 else np.zeros((M, N), np.float32)
        C = dev.put(C0)
    flags = (0x100 if ax2 else 0) | (0x200 if cx2 else 0)
    ok(vsl, H.vsl_gemm_f16(dev.p(dev.put(Ad)), dev.p(dev.put(B)), M, N, K, dev.p(C), epi | flags, None))
    out = dev.get(C).astype(np.float64)
    rows = np.unique(np.concatenate([[0, M - 1, M // 2], rng.integers(0, M, 40)]))
    prod = Aref[rows] @ B.astype(np.float64).T
    if epi == 3:
        ref = orc.swiglu(prod[:, :N].astype(np.float32).ravel(), prod[:, N:].astype(np.float32).ravel())
        ref = ref.reshape(len(rows), N)
        got = out[rows] + (out[M + rows] if cx2 else 0.0)
        assert rel_err(got, ref) < (2.0 ** -18 if cx2 else 2.0 ** -9)
    elif epi == 1:
        assert rel_err(out[rows], prod) < 2.0 ** -10
    else:
        ref = prod + (C0[rows] if epi == 2 else 0.0)
        assert rel_err(out[rows], ref) < 1e-5


@pytest.mark.parametrize("M,N,K,epi,ax2", [
    (512, 4096, 14336, 2, True),   # down projection of a 512-row chunk: residual add, split A
    (512, 6144, 4096, 0, True),    # QKV: fp32 store, 128 x 192 tiles (128 tiles x 2 chunks)
    (512, 1536, 4096, 0, False),   # one-plane A on 128 x 192 tiles (32 tiles x 8 chunks)
    (300, 6144, 4096, 2, True),    # ragged M on 128 x 192 tiles, residual add
    (512, 4096, 4096, 1, False),   # fp16 store
    (300, 4096, 2048, 2, False),   # ragged M
    (128, 2048, 8192, 2, True),    # 1B down projection of a 128-row prompt: 32 chunks of 256
    (128, 3072, 2048, 0, True),    # 1B QKV: 16 chunks of 128 reach 192 items
    (128, 2048, 2048, 2, False),   # 1B O projection: the widest split (16) short of 192 items
])
def test_gemm_splitk(vsl, dev, H, M, N, K, epi, ax2):
    """Narrow shapes through vsl_gemm_f16_ws: split over K into a workspace (128 x 256 tiles, or 128 x 192
    where whole rounds of those cost less), reduced in order with the epilogue; a too-small workspace
    runs unsplit with the same result (to rounding)."""
    rng = np.random.default_rng(M + N + K + epi)
    Af = rng.normal(0, 1, (M, K)).astype(np.float32)
    B = rng.normal(0, 0.02, (N, K)).astype(np.float16)
    if ax2:
        hi = Af.astype(np.float16)
        lo = (Af - hi.astype(np.float32)).astype(np.float16)
        Ad, Aref = np.concatenate([hi, lo]), hi.astype(np.float64) + lo.astype(np.float64)
    else:
        Ad = Af.astype(np.float16)
        Aref = Ad.astype(np.float64)
    flags = epi | (0x100 if ax2 else 0)
    need = H.vsl_gemm_f16_ws_bytes(M, N, K, flags)
    assert need > 0 and need % (4 * M * N) == 0
    ws = dev.empty((need // 4 + 4,), np.float32)
    C0 = rng.normal(0, 1, (M, N)).astype(np.float32) if epi == 2 else np.zeros((M, N), np.float32)
    outs = []
    for ws_bytes in (need, need - 4):  # the second call runs unsplit
        C = dev.empty((M, N), np.float16) if epi == 1 else dev.put(C0)
        ok(vsl, H.vsl_gemm_f16_ws(dev.p(dev.put(Ad)), dev.p(dev.put(B)), M, N, K, dev.p(C), flags, dev.p(ws),
                                  ws_bytes, None))
        outs.append(dev.get(C).astype(np.float64))
    rows = np.unique(np.concatenate([[0, M - 1], rng.integers(0, M, 40)]))
    ref = Aref[rows] @ B.astype(np.float64).T + (C0[rows] if epi == 2 else 0.0)
    for out in outs:
        assert rel_err(out[rows], ref) < (2.0 ** -10 if epi == 1 else 1e-5)
    # a shape that fills the chip with whole tiles needs no workspace
    assert H.vsl_gemm_f16_ws_bytes(2048, 6144, 4096, 0) == 0


def test_gemm_f16_swiglu(vsl, orc, dev, H):
    rng = np.random.default_rng(21)
    M, F, K = 130, 512, 2048
    A = rng.normal(0, 1, (M, K)).astype(np.float16)
    B = rng.normal(0, 0.02, (2 * F, K)).astype(np.float16)
    C = dev.empty((M, F), np.float16)
    ok(vsl, H.vsl_gemm_f16(dev.p(dev.put(A)), dev.p(dev.put(B)), M, F, K, dev.p(C), 3, None))
    gu = A.astype(np.float64) @ B.astype(np.float64).T
    ref = orc.swiglu(gu[:, :F].astype(np.float32).ravel(), gu[:, F:].astype(np.float32).ravel()).reshape(M, F)
    assert rel_err(dev.get(C).astype(np.float32), ref) < 2.0 ** -9


@pytest.mark.parametrize("M,N,K,epi,ax2", [
    (128, 8192, 2048, 3, True),     # 1B gate/up of a 128-row prompt: 2 x 128 tiles of 64 x (64 + 64)
    (100, 8192, 2048, 3, False),    # ragged M, one-plane A
    (128, 16384, 2048, 0, True),    # fp32 store without a workspace: 2 x 128 tiles of 64 x 128
])
def test_gemm_small_rows(vsl, orc, dev, H, M, N, K, epi, ax2):
    """Few-row shapes that reach neither 192 tiles of 128 x 256 nor a K split (no workspace) run the
    64 x 128 direct-to-LDS tiles: against the fp64 product (SwiGLU applied in fp64)."""
    rng = np.random.default_rng(M + N + K)
    Af = rng.normal(0, 1, (M, K)).astype(np.float32)
    nb = 2 * N if epi == 3 else N
    B = rng.normal(0, 0.02, (nb, K)).astype(np.float16)
    if ax2:
        hi = Af.astype(np.float16)
        lo = (Af - hi.astype(np.float32)).astype(np.float16)
        Ad, Aref = np.concatenate([hi, lo]), hi.astype(np.float64) + lo.astype(np.float64)
    else:
        Ad = Af.astype(np.float16)
        Aref = Ad.astype(np.float64)
    flags = epi | (vsl.GEMM_A_X2 if ax2 else 0)
    C = dev.empty((M, N), np.float16 if epi == 3 else np.float32)
    ok(vsl, H.vsl_gemm_f16(dev.p(dev.put(Ad)), dev.p(dev.put(B)), M, N, K, dev.p(C), flags, None))
    rows = np.unique(np.concatenate([[0, M - 1], rng.integers(0, M, 24)]))
    prod = Aref[rows] @ B.astype(np.float64).T
    out = dev.get(C).astype(np.float64)[rows]
    if epi == 3:
        ref = prod[:, :N] / (1.0 + np.exp(-prod[:, :N])) * prod[:, N:]
        assert rel_err(out, ref) < 2.0 ** -10
    else:
        assert rel_err(out, prod) < 1e-5


@pytest.mark.parametrize("hd,nq,nkv,S,pos0", [(128, 32, 8, 77, 0), (128, 32, 8, 64, 100), (64, 32, 8, 200, 0),
                                              (64, 8, 8, 33, 5), (128, 32, 8, 1, 0), (128, 16, 8, 1, 300),
                                              (64, 16, 2, 5, 40), (128, 24, 8, 77, 3), (64, 15, 3, 40, 0),
                                              (128, 12, 2, 100, 9), (64, 14, 2, 33, 0)])
def test_rope_split_and_attn_prefill(vsl, orc, dev, H, hd, nq, nkv, S, pos0):
    rng = np.random.default_rng(hd + S + pos0)
    cap, theta = 512, 10000.0
    W = (nq + 2 * nkv) * hd
    qkv = rng.normal(0, 1, (S, W)).astype(np.float32)
    cs, sn = rope_tables(cap, hd, theta)
    K0 = rng.normal(0, 1, (nkv, cap, hd)).astype(np.float16)
    V0 = rng.normal(0, 1, (nkv, cap, hd)).astype(np.float16)
    kc, vc = dev.put(K0), dev.put(V0)
    q = dev.empty((S, nq * hd), np.float16)
    ok(vsl, H.vsl_rope_split_append(dev.p(dev.put(qkv)), S, nq, nkv, hd, pos0, dev.p(dev.put(cs)), dev.p(dev.put(sn)),
                                    dev.p(q), 1, dev.p(kc), dev.p(vc), 1, cap, None))
    K = dev.get(kc).astype(np.float32)
    V = dev.get(vc).astype(np.float32)
    Q = dev.get(q).astype(np.float32)
    for s in (0, S // 2, S - 1):
        pos = pos0 + s
        qr = orc.rope(qkv[s, :nq * hd], nq, hd, pos, theta)
        kr = orc.rope(qkv[s, nq * hd:(nq + nkv) * hd], nkv, hd, pos, theta)
        assert rel_err(Q[s], qr) < 2.0 ** -10
        assert rel_err(K[:, pos].reshape(-1), kr) < 2.0 ** -10
        assert rel_err(V[:, pos].reshape(-1), qkv[s, (nq + nkv) * hd:]) < 2.0 ** -10
    assert np.array_equal(K[:, :pos0], K0[:, :pos0].astype(np.float32))
    out = dev.empty((S, nq * hd), np.float16)
    scale = 1.0 / math.sqrt(hd)
    ok(vsl, H.vsl_attn_prefill(dev.p(q), 1, dev.p(kc), dev.p(vc), S, pos0, nq, nkv, hd, cap, scale, dev.p(out), 1,
                               None))
    O = dev.get(out).astype(np.float32)
    for s in range(0, S, max(1, S // 9)):
        ref = orc.attention_decode(Q[s], K, V, nq, nkv, hd, cap, pos0 + s + 1, scale)
        # P is rounded to fp16 before the PV product and the output is fp16
        assert rel_err(O[s], ref) < 4e-3


# ------------------------------------------------------------------------------------------
# runtime: synthetic fill, arena, graphs
# ------------------------------------------------------------------------------------------
def test_fill_normal_matches_host_generator(vsl, orc, dev, H):
    n = 1000003
    d16 = dev.empty((n,), np.float16)
    ok(vsl, H.vsl_fill_normal(dev.p(d16), 1, n, 3, b"blk.0.attn_q.weight", 0.0, 0.02, None))
    ref16 = orc.fill_normal(n, orc.F16, 3, "blk.0.attn_q.weight")
    d = dev.get(d16).view(np.uint16).astype(np.int64) - ref16.view(np.uint16).astype(np.int64)
    # device fp64 log/sin/cos may differ from the host's in the last bit; after two roundings that
    # reaches the fp16 value for at most a handful of elements, by one ulp
    assert np.count_nonzero(d) <= 8 and np.max(np.abs(d)) <= 1
    d32 = dev.empty((n,), np.float32)
    ok(vsl, H.vsl_fill_normal(dev.p(d32), 0, n, 3, b"x", 0.0, 1.0, None))
    ref32 = orc.fill_normal(n, orc.F32, 3, "x", 0.0, 1.0)
    g = dev.get(d32)
    # fp64 log/sin/cos may differ in the last bit between libraries; after rounding to fp32 that
    # shows up in at most a few elements, by one fp32 ulp
    diff = g.view(np.uint32).astype(np.int64) - ref32.view(np.uint32).astype(np.int64)
    assert np.count_nonzero(diff) <= 8 and np.max(np.abs(diff)) <= 1


def test_arena_suballocation(vsl, H):
    a = ctypes.c_void_p()
    ok(vsl, H.vsl_arena_create(0, 1 << 24, ctypes.byref(a)))
    try:
        ptrs = []
        for sz in (1000, 1 << 20, 256, 5 << 20):
            p = ctypes.c_void_p()
            ok(vsl, H.vsl_arena_alloc(a, sz, 256, ctypes.byref(p)))
            assert p.value % 256 == 0
            ptrs.append(p)
        st = vsl.PoolStats()
        ok(vsl, H.vsl_arena_stats(a, ctypes.byref(st)))
        assert st.allocation_count == 4 and st.used_size == 1024 + (1 << 20) + 256 + (5 << 20)
        ok(vsl, H.vsl_arena_free(a, ptrs[1]))
        ok(vsl, H.vsl_arena_free(a, ptrs[2]))
        p = ctypes.c_void_p()
        ok(vsl, H.vsl_arena_alloc(a, (1 << 20) + 256, 256, ctypes.byref(p)))
        assert p.value == ptrs[1].value  # coalesced hole reused first-fit
        big = ctypes.c_void_p()
        assert H.vsl_arena_alloc(a, 1 << 25, 256, ctypes.byref(big)) == -102
        ok(vsl, H.vsl_arena_reset(a))
        ok(vsl, H.vsl_arena_stats(a, ctypes.byref(st)))
        assert st.used_size == 0 and st.allocation_count == 0
    finally:
        H.vsl_arena_destroy(a)


def test_graph_replay_matches_eager(vsl, orc, dev, H):
    """A captured residual GEMV replayed several times, with eager work and syncs in between."""
    rng = np.random.default_rng(30)
    d, K = 1024, 2048
    W = dev.put(rng.normal(0, 0.02, (d, K)).astype(np.float16))
    x = dev.put(rng.normal(0, 1, K).astype(np.float32))
    r0 = rng.normal(0, 1, d).astype(np.float32)
    r = dev.put(r0)
    st = ctypes.c_void_p()
    ok(vsl, H.vsl_stream_create(ctypes.byref(st)))
    g = ctypes.c_void_p()
    ok(vsl, H.vsl_graph_begin(st))
    ok(vsl, H.vsl_gemv_residual(dev.p(W), 1, d, K, dev.p(x), dev.p(r), None, st))
    ok(vsl, H.vsl_graph_end(st, ctypes.byref(g)))
    dev.sync()
    assert np.array_equal(dev.get(r), r0)  # capture does not execute
    eager = dev.empty((d,), np.float32)
    inc = orc.gemm_nt(dev.get(W), dev.get(x))[:, 0]
    for i in range(1, 4):
        ok(vsl, H.vsl_graph_launch(g, st))
        ok(vsl, H.vsl_stream_sync(st))
        ok(vsl, H.vsl_gemv_residual(dev.p(W), 1, d, K, dev.p(x), dev.p(eager), None, None))
        dev.sync()
        assert rel_err(dev.get(r), r0 + i * inc) < 1e-5
    ok(vsl, H.vsl_graph_destroy(g))
    ok(vsl, H.vsl_stream_destroy(st))


# ------------------------------------------------------------------------------------------
# split (hi/lo fp16) activations on the prefill path
# ------------------------------------------------------------------------------------------
def split_np(a):
    hi = a.astype(np.float16)
    lo = (a - hi.astype(np.float32)).astype(np.float16)
    return hi, lo


def test_rmsnorm_split_planes(vsl, orc, dev, H):
    rng = np.random.default_rng(40)
    rows, d = 7, 4096
    x = rng.normal(0, 2, (rows, d)).astype(np.float32)
    g = rng.normal(1, 0.1, d).astype(np.float32)
    out = dev.empty((2, rows, d), np.float16)
    ok(vsl, H.vsl_rmsnorm(dev.p(dev.put(x)), dev.p(dev.put(g)), rows, d, 1e-5, dev.p(out), vsl.VSL_DT_F16X2, None))
    o = dev.get(out).astype(np.float32)
    ref = np.stack([orc.rmsnorm(x[r], g, 1e-5) for r in range(rows)])
    assert rel_err(o[0] + o[1], ref) < 2e-6  # hi + lo reproduces the fp32 value
    assert np.array_equal(o[0], ref.astype(np.float16).astype(np.float32)) or rel_err(o[0], ref) < 2.0 ** -11


@pytest.mark.parametrize("d", [256, 512, 1024, 2048, 4096, 8192, 1000])
@pytest.mark.parametrize("rows", [1, 6])
@pytest.mark.parametrize("odt", [0, 1, 2])
def test_rmsnorm_rows_widths(vsl, orc, dev, H, d, rows, odt):
    """Row RMSNorm for every width the one-row-per-wave kernel holds in registers (256 .. 8192) and a
    width that takes the block-per-row kernel (1000), row counts that leave waves of a block without
    a row, fp32 / fp16 / split outputs, with and without gains. The split reproduces the fp32 result
    and its hi plane is a nearest binary16 of hi + lo."""
    rng = np.random.default_rng(d + rows + 7 * odt)
    x = rng.normal(0, 2, (rows, d)).astype(np.float32)
    g = rng.normal(1, 0.1, d).astype(np.float32) if odt != 1 else None
    planes = 2 if odt == 2 else 1
    out = dev.empty((planes, rows, d), np.float32 if odt == 0 else np.float16)
    ok(vsl, H.vsl_rmsnorm(dev.p(dev.put(x)), dev.p(dev.put(g)) if g is not None else None, rows, d, 1e-5, dev.p(out),
                          odt, None))
    o = dev.get(out).astype(np.float64)
    gg = g if g is not None else np.ones(d, np.float32)
    ref = np.stack([orc.rmsnorm(x[r], gg, 1e-5) for r in range(rows)]).astype(np.float64)
    if odt == 0:
        assert rel_err(o[0], ref) < 2e-6
    elif odt == 1:
        assert rel_err(o[0], ref) < 2.0 ** -11
    else:
        assert rel_err(o[0] + o[1], ref) < 2e-6
        # hi is a nearest binary16 of hi + lo: |lo| is at most half the fp16 spacing at hi (a split
        # whose stored hi came from a different rounding than lo leaves up to a whole spacing)
        hi16 = o[0].astype(np.float16)
        assert np.all(np.abs(o[1]) <= 0.5 * np.spacing(np.abs(hi16)).astype(np.float64))


@pytest.mark.parametrize("M,N,K,epi", [(77, 256, 4096, 0), (130, 512, 2048, 2), (200, 4096, 14336, 2)])
def test_gemm_split_a(vsl, dev, H, M, N, K, epi):
    rng = np.random.default_rng(M + N + K)
    A = rng.normal(0, 1, (M, K)).astype(np.float32)
    B = rng.normal(0, 0.02, (N, K)).astype(np.float16)
    hi, lo = split_np(A)
    ref = A.astype(np.float64) @ B.astype(np.float64).T
    C0 = rng.normal(0, 1, (M, N)).astype(np.float32) if epi == 2 else np.zeros((M, N), np.float32)
    C = dev.put(C0)
    ok(vsl, H.vsl_gemm_f16(dev.p(dev.put(np.stack([hi, lo]))), dev.p(dev.put(B)), M, N, K, dev.p(C),
                           epi | vsl.GEMM_A_X2, None))
    # the split input is accurate to ~2^-22 relative: the result matches the fp32-input product
    assert rel_err(dev.get(C).astype(np.float64) - C0, ref) < 5e-6


def test_gemm_swiglu_split_in_out(vsl, orc, dev, H):
    rng = np.random.default_rng(41)
    M, F, K = 130, 512, 2048
    A = rng.normal(0, 1, (M, K)).astype(np.float32)
    B = rng.normal(0, 0.02, (2 * F, K)).astype(np.float16)
    hi, lo = split_np(A)
    C = dev.empty((2, M, F), np.float16)
    ok(vsl, H.vsl_gemm_f16(dev.p(dev.put(np.stack([hi, lo]))), dev.p(dev.put(B)), M, F, K, dev.p(C),
                           3 | vsl.GEMM_A_X2 | vsl.GEMM_C_X2, None))
    gu = A.astype(np.float64) @ B.astype(np.float64).T
    ref = orc.swiglu(gu[:, :F].astype(np.float32).ravel(), gu[:, F:].astype(np.float32).ravel()).reshape(M, F)
    c = dev.get(C).astype(np.float32)
    assert rel_err(c[0] + c[1], ref) < 2e-6


@pytest.mark.parametrize("hd,nq,nkv,S,pos0", [(128, 32, 8, 77, 0), (64, 32, 8, 64, 100), (128, 32, 8, 1056, 0)])
def test_attn_prefill_split(vsl, orc, dev, H, hd, nq, nkv, S, pos0):
    """Split q / split output prefill attention against the oracle. Fewer than 256 blocks of (32 rows,
    KV head) split each group of four query heads over two blocks; 1056 rows on 8 KV heads (264 blocks)
    keep one block per group."""
    rng = np.random.default_rng(hd + S + pos0 + 1)
    cap, theta = max(512, pos0 + S), 10000.0
    W = (nq + 2 * nkv) * hd
    qkv = rng.normal(0, 1, (S, W)).astype(np.float32)
    cs, sn = rope_tables(cap, hd, theta)
    kc = dev.put(rng.normal(0, 1, (nkv, cap, hd)).astype(np.float16))
    vc = dev.put(rng.normal(0, 1, (nkv, cap, hd)).astype(np.float16))
    q = dev.empty((2, S, nq * hd), np.float16)
    ok(vsl, H.vsl_rope_split_append(dev.p(dev.put(qkv)), S, nq, nkv, hd, pos0, dev.p(dev.put(cs)), dev.p(dev.put(sn)),
                                    dev.p(q), vsl.VSL_DT_F16X2, dev.p(kc), dev.p(vc), 1, cap, None))
    Q = dev.get(q).astype(np.float32)
    Qf = Q[0] + Q[1]
    for s in (0, S - 1):
        assert rel_err(Qf[s], orc.rope(qkv[s, :nq * hd], nq, hd, pos0 + s, theta)) < 2e-6
    out = dev.empty((2, S, nq * hd), np.float16)
    scale = 1.0 / math.sqrt(hd)
    ok(vsl, H.vsl_attn_prefill(dev.p(q), vsl.VSL_DT_F16X2, dev.p(kc), dev.p(vc), S, pos0, nq, nkv, hd, cap, scale,
                               dev.p(out), vsl.VSL_DT_F16X2, None))
    O = dev.get(out).astype(np.float32)
    K = dev.get(kc).astype(np.float32)
    V = dev.get(vc).astype(np.float32)
    for s in range(0, S, max(1, S // 7)):
        ref = orc.attention_decode(Qf[s], K, V, nq, nkv, hd, cap, pos0 + s + 1, scale)
        assert rel_err(O[0][s] + O[1][s], ref) < 2e-5


# ------------------------------------------------------------------------------------------
# prefill projections fused with the step that consumes them
# ------------------------------------------------------------------------------------------
def _act(rng, M, K, ax2):
    """fp16 activations (or split hi/lo planes) and the fp64 values they stand for."""
    Af = rng.normal(0, 1, (M, K)).astype(np.float32)
    if ax2:
        hi, lo = split_np(Af)
        return np.concatenate([hi, lo]), hi.astype(np.float64) + lo.astype(np.float64)
    Ad = Af.astype(np.float16)
    return Ad, Ad.astype(np.float64)


@pytest.mark.parametrize("S,K,nq,nkv,hd,pos0,ax2,qx2,kvdt", [
    (512, 4096, 32, 8, 128, 0, True, True, 1),     # 512-row chunk of the 8B-class model: K split 2
    (512, 4096, 32, 8, 128, 100, False, False, 1),  # later chunk, fp16 q
    (300, 4096, 32, 8, 128, 7, True, True, 0),     # ragged rows (K split 4), fp32 cache
    (256, 4096, 32, 8, 64, 0, False, True, 1),     # head_dim 64 (K split 8)
    (128, 2048, 32, 8, 64, 0, True, True, 1),      # 1B 128-row prompt: K split 16 (runtime-count sum)
])
def test_gemm_qkv_rope_append(vsl, orc, dev, H, S, K, nq, nkv, hd, pos0, ax2, qx2, kvdt):
    """QKV projection + RoPE + Q/K/V split through one entry point. With the workspace the split-K
    partials are summed, rotated and stored by one launch: its q, k and v equal those of the unfused
    composition (the projection into an fp32 buffer through the same workspace, then
    vsl_rope_split_append) exactly, since both add the same partials in the same order, and match the
    oracle's RoPE of the fp64 projection. Without the workspace the entry runs unsplit through the
    buffer. Cache positions outside pos0..pos0+S-1 are left alone."""
    rng = np.random.default_rng(S + hd + pos0)
    cap, theta = 1024, 500000.0
    N = (nq + 2 * nkv) * hd
    Ad, Aref = _act(rng, S, K, ax2)
    W = rng.normal(0, 0.02, (N, K)).astype(np.float16)
    cs, sn = rope_tables(cap, hd, theta)
    kvnp = np.float16 if kvdt == 1 else np.float32
    K0 = rng.normal(0, 1, (nkv, cap, hd)).astype(kvnp)
    need = H.vsl_gemm_f16_ws_bytes(S, N, K, 0)
    assert need > 0
    ws = dev.empty((need // 4,), np.float32)
    dA, dW, dcs, dsn = dev.put(Ad), dev.put(W), dev.put(cs), dev.put(sn)
    qkv = dev.empty((S, N), np.float32)
    qdt, aflag = (2 if qx2 else 1), (0x100 if ax2 else 0)
    outs = []
    for mode in ("fused", "unfused", "unsplit"):
        q = dev.empty(((2 if qx2 else 1) * S, nq * hd), np.float16)
        kc, vc = dev.put(K0), dev.put(K0)
        if mode == "unfused":
            ok(vsl, H.vsl_gemm_f16_ws(dev.p(dA), dev.p(dW), S, N, K, dev.p(qkv), aflag, dev.p(ws), need, None))
            ok(vsl, H.vsl_rope_split_append(dev.p(qkv), S, nq, nkv, hd, pos0, dev.p(dcs), dev.p(dsn), dev.p(q), qdt,
                                            dev.p(kc), dev.p(vc), kvdt, cap, None))
        else:
            ok(vsl, H.vsl_gemm_f16_qkv_rope_append(dev.p(dA), dev.p(dW), S, K, aflag, nq, nkv, hd, pos0, dev.p(dcs),
                                                   dev.p(dsn), dev.p(q), qdt, dev.p(kc), dev.p(vc), kvdt, cap,
                                                   dev.p(qkv), dev.p(ws) if mode == "fused" else None,
                                                   need if mode == "fused" else 0, None))
        outs.append((dev.get(q).astype(np.float64), dev.get(kc).astype(np.float64), dev.get(vc).astype(np.float64)))
    for a, b in zip(outs[0], outs[1]):
        assert np.array_equal(a, b)
    for q, kc, vc in (outs[0], outs[2]):
        Q = (q[:S] + q[S:]) if qx2 else q
        outside = np.ones(cap, bool)
        outside[pos0:pos0 + S] = False
        assert np.array_equal(kc[:, outside], K0[:, outside].astype(np.float64))
        assert np.array_equal(vc[:, outside], K0[:, outside].astype(np.float64))
        qt = 2e-5 if qx2 else 2.0 ** -10
        kt = 2.0 ** -10 if kvdt == 1 else 2e-5
        for s in (0, 1, S // 2, S - 1):
            y = (Aref[s] @ W.astype(np.float64).T).astype(np.float32)
            pos = pos0 + s
            assert rel_err(Q[s], orc.rope(y[:nq * hd], nq, hd, pos, theta)) < qt
            assert rel_err(kc[:, pos].reshape(-1), orc.rope(y[nq * hd:(nq + nkv) * hd], nkv, hd, pos, theta)) < kt
            assert rel_err(vc[:, pos].reshape(-1), y[(nq + nkv) * hd:]) < kt


def test_gemm_qkv_rope_append_refuses_before_launch(vsl, dev, H):
    """Capacity and dtype errors come back as codes with nothing written."""
    S, K, nq, nkv, hd, cap = 64, 512, 4, 4, 64, 80
    N = (nq + 2 * nkv) * hd
    A = dev.put(np.zeros((S, K), np.float16))
    W = dev.put(np.zeros((N, K), np.float16))
    t = dev.put(np.zeros((cap, hd // 2), np.float32))
    q = dev.empty((S, nq * hd), np.float16)
    K0 = np.full((nkv, cap, hd), 3.0, np.float16)
    kc = dev.put(K0)
    qkv = dev.empty((S, N), np.float32)
    args = lambda pos0, qdt, kvdt: (dev.p(A), dev.p(W), S, K, 0, nq, nkv, hd, pos0, dev.p(t), dev.p(t), dev.p(q), qdt,
                                    dev.p(kc), dev.p(kc), kvdt, cap, dev.p(qkv), None, 0, None)
    assert H.vsl_gemm_f16_qkv_rope_append(*args(cap - S + 1, 1, 1)) == vsl.VSL_E_CAPACITY
    assert H.vsl_gemm_f16_qkv_rope_append(*args(0, 0, 1)) == vsl.VSL_E_UNSUPPORTED
    assert H.vsl_gemm_f16_qkv_rope_append(*args(0, 1, 5)) == vsl.VSL_E_UNSUPPORTED
    assert np.array_equal(dev.get(kc), K0)


@pytest.mark.parametrize("M,N,K,ax2,odt,gam", [
    (512, 4096, 4096, True, 2, True),    # O projection of a 512-row chunk + FFN norm (split planes)
    (512, 4096, 14336, True, 2, True),   # down projection + next layer's attention norm
    (300, 4096, 4096, False, 1, True),   # ragged rows, fp16 out
    (512, 2048, 8192, False, 0, False),  # d = 2048, K split 8, fp32 out, no gains
    (256, 8192, 4096, False, 2, True),   # d = 8192 (eight float4 per thread)
    (128, 2048, 8192, True, 2, True),    # 1B down projection of a 128-row prompt: K split 32
    (128, 2048, 2048, False, 1, True),   # 1B O projection: K split 16
])
def test_gemm_resid_rmsnorm(vsl, orc, dev, H, M, N, K, ax2, odt, gam):
    """Residual projection + the next RMSNorm through one entry point. With the workspace the split-K
    partials are summed and added to x, and the rows normalized, by one launch: x equals the unfused
    residual GEMM's exactly (same partials, same order) and the fp64 reference to fp32 rounding; the
    norm matches the oracle's RMSNorm of the updated x. Without the workspace the entry runs the
    unsplit residual GEMM and vsl_rmsnorm."""
    rng = np.random.default_rng(M + N + K + odt)
    Ad, Aref = _act(rng, M, K, ax2)
    B = rng.normal(0, 0.02, (N, K)).astype(np.float16)
    x0 = rng.normal(0, 1, (M, N)).astype(np.float32)
    g = rng.normal(1, 0.1, N).astype(np.float32) if gam else None
    need = H.vsl_gemm_f16_ws_bytes(M, N, K, 2)
    assert need > 0
    ws = dev.empty((need // 4,), np.float32)
    dA, dB = dev.put(Ad), dev.put(B)
    dg = dev.put(g) if gam else None
    aflag = 0x100 if ax2 else 0
    planes = 2 if odt == 2 else 1
    res = {}
    for mode in ("fused", "unfused", "unsplit"):
        x = dev.put(x0)
        xn = dev.empty((planes, M, N), np.float32 if odt == 0 else np.float16)
        if mode == "unfused":
            ok(vsl, H.vsl_gemm_f16_ws(dev.p(dA), dev.p(dB), M, N, K, dev.p(x), 2 | aflag, dev.p(ws), need, None))
        else:
            ok(vsl, H.vsl_gemm_f16_resid_rmsnorm(dev.p(dA), dev.p(dB), M, N, K, aflag, dev.p(x),
                                                 dev.p(dg) if gam else None, 1e-5, dev.p(xn), odt,
                                                 dev.p(ws) if mode == "fused" else None,
                                                 need if mode == "fused" else 0, None))
        res[mode] = (dev.get(x).astype(np.float32), dev.get(xn).astype(np.float64))
    assert np.array_equal(res["fused"][0], res["unfused"][0])
    rows = np.unique(np.concatenate([[0, M - 1], rng.integers(0, M, 24)]))
    ref = x0[rows].astype(np.float64) + Aref[rows] @ B.astype(np.float64).T
    gg = g if gam else np.ones(N, np.float32)
    for mode in ("fused", "unsplit"):
        x, o = res[mode]
        assert rel_err(x[rows], ref) < 1e-5
        nref = np.stack([orc.rmsnorm(x[r], gg, 1e-5) for r in rows]).astype(np.float64)
        if odt == 0:
            assert rel_err(o[0][rows], nref) < 2e-6
        elif odt == 1:
            assert rel_err(o[0][rows], nref) < 2.0 ** -11
        else:
            assert rel_err(o[0][rows] + o[1][rows], nref) < 2e-6
            hi16 = o[0][rows].astype(np.float16)
            assert np.all(np.abs(o[1][rows]) <= 0.5 * np.spacing(np.abs(hi16)).astype(np.float64))


def test_gemm_resid_rmsnorm_bad_arguments(vsl, dev, H):
    A = dev.put(np.zeros((8, 512), np.float16))
    x = dev.put(np.zeros((8, 1024), np.float32))
    xn = dev.empty((8, 1024), np.float16)
    assert H.vsl_gemm_f16_resid_rmsnorm(dev.p(A), dev.p(A), 8, 1024, 512, 0, dev.p(x), None, 1e-5, dev.p(xn), 7,
                                        None, 0, None) == vsl.VSL_E_UNSUPPORTED
    assert H.vsl_gemm_f16_resid_rmsnorm(dev.p(A), dev.p(A), 8, 1024, 512, 0x200, dev.p(x), None, 1e-5, dev.p(xn), 1,
                                        None, 0, None) == vsl.VSL_E_INVALID
    assert H.vsl_gemm_f16_resid_rmsnorm(dev.p(A), None, 8, 1024, 512, 0, dev.p(x), None, 1e-5, dev.p(xn), 1,
                                        None, 0, None) == vsl.VSL_E_INVALID


def test_fused_prefill_entries_misaligned_outputs(vsl, orc, dev, H):
    """Output buffers that are not 8-byte aligned take the unfused kernels (scalar RoPE split, residual
    GEMM + row RMSNorm); their results agree with the aligned fused path: residual rows exactly,
    normalized rows and q / k / v to fp32 rounding."""
    rng = np.random.default_rng(99)
    S, K, nq, nkv, hd, pos0, cap = 512, 4096, 32, 8, 128, 3, 1024
    N = (nq + 2 * nkv) * hd
    Ad, _ = _act(rng, S, K, True)
    W = rng.normal(0, 0.02, (N, K)).astype(np.float16)
    cs, sn = rope_tables(cap, hd, 500000.0)
    need = max(H.vsl_gemm_f16_ws_bytes(S, N, K, 0), H.vsl_gemm_f16_ws_bytes(S, 4096, K, 2))
    ws = dev.empty((need // 4,), np.float32)
    dA, dW, dcs, dsn = dev.put(Ad), dev.put(W), dev.put(cs), dev.put(sn)
    qkv = dev.empty((S, N), np.float32)
    res = []
    for off in (0, 2):  # byte offset of q_out: 0 (fused path) or 2 (scalar fallback)
        qbuf = dev.empty((2 * S * nq * hd + 8,), np.float16)
        kc, vc = dev.empty((nkv, cap, hd), np.float16), dev.empty((nkv, cap, hd), np.float16)
        ok(vsl, H.vsl_gemm_f16_qkv_rope_append(dev.p(dA), dev.p(dW), S, K, 0x100, nq, nkv, hd, pos0, dev.p(dcs),
                                               dev.p(dsn), dev.p(qbuf) + off, 2, dev.p(kc), dev.p(vc), 1, cap,
                                               dev.p(qkv), dev.p(ws), need, None))
        q = dev.get(qbuf).view(np.uint8)[off:off + 2 * S * nq * hd * 2].view(np.float16).astype(np.float64)
        res.append((q[:S * nq * hd] + q[S * nq * hd:], dev.get(kc).astype(np.float64), dev.get(vc).astype(np.float64)))
    assert rel_err(res[1][0], res[0][0]) < 1e-6  # q as hi + lo carries the fp32 value
    for a, b in zip(res[0][1:], res[1][1:]):
        assert rel_err(b, a) < 2.0 ** -10  # fp16 caches: a last-bit fp32 difference can flip a rounding
    # residual + RMSNorm into a misaligned fp16 output
    B = rng.normal(0, 0.02, (4096, K)).astype(np.float16)
    x0 = rng.normal(0, 1, (S, 4096)).astype(np.float32)
    g = rng.normal(1, 0.1, 4096).astype(np.float32)
    dB, dg = dev.put(B), dev.put(g)
    out = []
    for off in (0, 2):
        x = dev.put(x0)
        xbuf = dev.empty((S * 4096 + 8,), np.float16)
        ok(vsl, H.vsl_gemm_f16_resid_rmsnorm(dev.p(dA), dev.p(dB), S, 4096, K, 0x100, dev.p(x), dev.p(dg), 1e-5,
                                             dev.p(xbuf) + off, 1, dev.p(ws), need, None))
        xn = dev.get(xbuf).view(np.uint8)[off:off + S * 4096 * 2].view(np.float16).astype(np.float64)
        out.append((dev.get(x), xn))
    assert np.array_equal(out[0][0], out[1][0])
    assert rel_err(out[1][1], out[0][1]) < 2.0 ** -10
