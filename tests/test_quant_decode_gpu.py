"""Resident block-quantized packs (VSL_DT_Q8_0 / Q4_0 / Q4_1) in the decode GEMVs.

A pack built from GGUF blocks (both block layouts, the reference's scale special cases included)
dequantizes back to the oracle's dequantized values bit for bit, so its contents are pinned by the
oracle's orc_dequant (itself pinned in test_quant.py).  Every decode entry point over a pack is then
checked against the same op over those fp32 values: the GEMV against the fp64 product, the fused
residual / SwiGLU / QKV + RoPE + KV-append / lm_head epilogues against the fp32-weight launch of the
same entry point.  The on-device quantizer (synthetic models) is checked against its rounding bound."""
import numpy as np
import pytest

import vsl_testlib
from test_quant import GGML_IDS, REF_IDS, bits, dq, np_quantize

pytestmark = pytest.mark.gpu

WF = {"q4_0": 2, "q4_1": 3, "q8_0": 4}
DT = {"q8_0": 4, "q4_0": 5, "q4_1": 6}
FMTS = ["q8_0", "q4_0", "q4_1"]


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
    return float(np.max(np.abs(a - b)) / max(np.max(np.abs(b)), 1e-30))


def _raw(fmt, conv, rows, K, seed, scale=0.05):
    rng = np.random.default_rng(seed)
    return np_quantize((rng.standard_normal(rows * K) * scale).astype(np.float32), fmt, conv)


def _values(orc, raw, fmt, conv, n):
    r, v = dq(orc, raw, (REF_IDS if conv == 0 else GGML_IDS)[fmt], conv, n)
    assert r == n
    return v[:n]


def _pack(vsl, H, dev, parts, fmt, conv, K):
    """One pack holding the row blocks of `parts` (raw GGUF block bytes, rows each) stacked in order."""
    rows = sum(r for r, _ in parts)
    pack = dev.empty((H.vsl_quant_pack_bytes(DT[fmt], rows, K),), np.uint8)
    assert dev.p(pack) % 256 == 0
    b0 = 0
    for r, raw in parts:
        src = dev.put(np.frombuffer(raw, np.uint8))
        ok(vsl, H.vsl_quant_pack(dev.p(src), WF[fmt], conv, r * K // 32, dev.p(pack), rows, K, b0, None))
        b0 += r * K // 32
    return pack


@pytest.mark.parametrize("fmt", FMTS)
@pytest.mark.parametrize("conv", [0, 1])
def test_pack_holds_the_dequantized_values(vsl, orc, dev, H, fmt, conv):
    """Two tensors packed as consecutive rows of one pack (as [Wq; Wk; Wv] is) dequantize to the
    oracle's values bit for bit, including blocks whose scales the reference's helper treats specially
    (negative subnormal, -0, smallest subnormal) and a large one; pack sizes by formula."""
    import struct
    K, r1, r2 = 96, 40, 13
    raw1 = bytearray(_raw(fmt, conv, r1, K, 1))
    bb = {"q4_0": 18, "q4_1": 20, "q8_0": 34}[fmt]
    for i, sc in enumerate([0x8001, 0x8000, 0x0001, 0x83FF, 0x7BFF]):
        raw1[(7 * i + 2) * bb:(7 * i + 2) * bb + 2] = struct.pack("<H", sc)
    raw1 = bytes(raw1)
    raw2 = _raw(fmt, conv, r2, K, 2)
    pack = _pack(vsl, H, dev, [(r1, raw1), (r2, raw2)], fmt, conv, K)
    want = np.concatenate([_values(orc, raw1, fmt, conv, r1 * K), _values(orc, raw2, fmt, conv, r2 * K)])
    out = dev.empty(((r1 + r2) * K,), np.float32)
    ok(vsl, H.vsl_dequant_pack(dev.p(pack), DT[fmt], r1 + r2, K, dev.p(out), vsl.VSL_DT_F32, None))
    assert bits(dev.get(out)).tolist() == bits(want).tolist()
    out16 = dev.empty(((r1 + r2) * K,), np.float16)
    ok(vsl, H.vsl_dequant_pack(dev.p(pack), DT[fmt], r1 + r2, K, dev.p(out16), vsl.VSL_DT_F16, None))
    assert np.array_equal(dev.get(out16).view(np.uint16), want.astype(np.float16).view(np.uint16))
    rows, nb = r1 + r2, (r1 + r2) * K // 32
    vb = rows * K * (8 if fmt == "q8_0" else 4) // 8
    al = lambda b: (b + 255) // 256 * 256
    assert H.vsl_quant_pack_bytes(DT[fmt], rows, K) == al(vb) + al(4 * nb) * (2 if fmt == "q4_1" else 1)
    assert H.vsl_quant_pack_bytes(DT[fmt], rows, 100) == 0


@pytest.mark.parametrize("fmt", FMTS)
@pytest.mark.parametrize("N,K", [(1000, 4096), (4099, 2048), (300, 14336), (64, 28672), (7, 32)])
def test_quant_gemv(vsl, orc, dev, H, fmt, N, K):
    """y = W x at B = 1 over a pack (fp32 and fp16 y) against the fp64 product of the dequantized
    values: 2048 columns per tile in every format, wide K on the 16-wave blocks, one-block rows."""
    conv = 1 if fmt == "q4_0" else 0
    raw = _raw(fmt, conv, N, K, N + K)
    W = _values(orc, raw, fmt, conv, N * K).reshape(N, K).astype(np.float64)
    pack = _pack(vsl, H, dev, [(N, raw)], fmt, conv, K)
    x = np.random.default_rng(K).normal(0, 1, K).astype(np.float32)
    ref = W @ x.astype(np.float64)
    y = dev.empty((N,), np.float32)
    ok(vsl, H.vsl_gemv(dev.p(pack), DT[fmt], N, K, dev.p(dev.put(x)), vsl.VSL_DT_F32, 1, dev.p(y), vsl.VSL_DT_F32,
                       None))
    assert rel_err(dev.get(y), ref) < 1e-5
    y16 = dev.empty((N,), np.float16)
    ok(vsl, H.vsl_gemv(dev.p(pack), DT[fmt], N, K, dev.p(dev.put(x)), vsl.VSL_DT_F32, 1, dev.p(y16), vsl.VSL_DT_F16,
                       None))
    assert rel_err(dev.get(y16), ref) < 2.0 ** -10


@pytest.mark.parametrize("fmt", FMTS)
@pytest.mark.parametrize("N,K", [(4096, 14336), (300, 28672), (1000, 4096), (33, 96), (70, 32768), (8193, 8192)])
def test_quant_gemv_residual_shapes(vsl, dev, H, fmt, N, K):
    """The residual GEMV over a pack (the O / down projection; from 8192 columns on 16-wave blocks, two
    rows per wave from 8192 rows) against the pack's dequantized values in float64, at the 8B down
    shape, past 16384 columns, a short row, a row of one block and an odd row count past 8192. The
    pack comes from the device quantizer and the reference from its dequantized values (both pinned
    against the oracle's block arithmetic by the tests above), which keeps the large shapes cheap."""
    rng = np.random.default_rng(N + 7)
    w16 = (rng.standard_normal((N, K), dtype=np.float32) * 0.05).astype(np.float16)
    pack = dev.empty((H.vsl_quant_pack_bytes(DT[fmt], N, K),), np.uint8)
    ok(vsl, H.vsl_quantize_pack(dev.p(dev.put(w16)), vsl.VSL_DT_F16, N, K, DT[fmt], dev.p(pack), None))
    deq = dev.empty((N, K), np.float32)
    ok(vsl, H.vsl_dequant_pack(dev.p(pack), DT[fmt], N, K, dev.p(deq), vsl.VSL_DT_F32, None))
    W = dev.get(deq).astype(np.float64)
    h = rng.normal(0, 1, K).astype(np.float32)
    r = rng.normal(0, 1, N).astype(np.float32)
    y = dev.put(r)
    ok(vsl, H.vsl_gemv_residual(dev.p(pack), DT[fmt], N, K, dev.p(dev.put(h)), dev.p(y), None, None))
    want = r.astype(np.float64) + W @ h.astype(np.float64)
    assert rel_err(dev.get(y), want) < 1e-5


@pytest.mark.parametrize("fmt", FMTS)
def test_quant_decode_ops(vsl, orc, dev, H, fmt):
    """The fused decode entry points over a pack against the same launches over the pack's fp32
    values: residual GEMV, RMSNorm + [Wgate; Wup] + SwiGLU, RMSNorm + [Wq; Wk; Wv] + RoPE + KV append
    (fp16 cache), final norm + lm_head + greedy argmax + next embedding."""
    from test_kernels_gpu import ctrl_buf, rope_tables
    conv = 0
    d, F, nq, nkv, hd, V, cap = 512, 1024, 4, 2, 128, 3000, 64
    rng = np.random.default_rng(31)

    def both(rows, K, seed):
        raw = _raw(fmt, conv, rows, K, seed)
        w32 = _values(orc, raw, fmt, conv, rows * K)
        return _pack(vsl, H, dev, [(rows, raw)], fmt, conv, K), dev.put(w32)

    x = rng.normal(0, 1, d).astype(np.float32)
    g = rng.normal(1, 0.1, d).astype(np.float32)
    # residual GEMV (down projection shape)
    pk, w32 = both(d, F, 1)
    h = rng.normal(0, 1, F).astype(np.float32)
    r = rng.normal(0, 1, d).astype(np.float32)
    ra, rb = dev.put(r), dev.put(r)
    ok(vsl, H.vsl_gemv_residual(dev.p(pk), DT[fmt], d, F, dev.p(dev.put(h)), dev.p(ra), None, None))
    ok(vsl, H.vsl_gemv_residual(dev.p(w32), vsl.VSL_DT_F32, d, F, dev.p(dev.put(h)), dev.p(rb), None, None))
    assert rel_err(dev.get(ra), dev.get(rb)) < 1e-5
    # SwiGLU
    pk, w32 = both(2 * F, d, 2)
    ha, hb = dev.empty((F,), np.float32), dev.empty((F,), np.float32)
    ok(vsl, H.vsl_norm_swiglu(dev.p(dev.put(x)), dev.p(dev.put(g)), 1e-5, dev.p(pk), DT[fmt], d, F, dev.p(ha), None,
                              None))
    ok(vsl, H.vsl_norm_swiglu(dev.p(dev.put(x)), dev.p(dev.put(g)), 1e-5, dev.p(w32), vsl.VSL_DT_F32, d, F, dev.p(hb),
                              None, None))
    assert rel_err(dev.get(ha), dev.get(hb)) < 1e-4
    # QKV + RoPE + KV append
    nr = (nq + 2 * nkv) * hd
    pk, w32 = both(nr, d, 3)
    cs, sn = rope_tables(cap, hd, 10000.0)
    outs = []
    for W, dt in ((pk, DT[fmt]), (w32, vsl.VSL_DT_F32)):
        kc, vc = dev.empty((nkv, cap, hd), np.float16), dev.empty((nkv, cap, hd), np.float16)
        q = dev.empty((nq * hd,), np.float32)
        c = ctrl_buf(vsl, dev, H, 9, cap=cap)
        ok(vsl, H.vsl_qkv_rope_append(dev.p(dev.put(x)), dev.p(dev.put(g)), 1e-5, dev.p(W), dt, d, nq, nkv, hd,
                                      dev.p(dev.put(cs)), dev.p(dev.put(sn)), dev.p(kc), dev.p(vc), 1, cap, dev.p(q),
                                      dev.p(c), None))
        outs.append((dev.get(q), dev.get(kc)[:, 9].astype(np.float32), dev.get(vc)[:, 9].astype(np.float32)))
    for a, b in zip(*outs):
        assert rel_err(a, b) < 2.0 ** -10
    # final norm + lm_head + greedy argmax + next embedding
    pk, w32 = both(V, d, 4)
    E = rng.normal(0, 0.02, (V, d)).astype(np.float16)
    nb = H.vsl_lm_head_ws_blocks()
    res = []
    for W, dt in ((pk, DT[fmt]), (w32, vsl.VSL_DT_F32)):
        ws_v, ws_i = dev.empty((nb,), np.float32), dev.empty((nb,), np.int32)
        toks, logits = dev.empty((4,), np.int32), dev.empty((V,), np.float32)
        dx = dev.put(x)
        c = ctrl_buf(vsl, dev, H, 5, max_steps=3, cap=cap)
        ok(vsl, H.vsl_lm_head_sample(dev.p(dev.put(g)), 1e-5, dev.p(W), dt, V, d, dev.p(dx), dev.p(dev.put(E)), 1,
                                     dev.p(logits), vsl.Sampler(0, 0.0, 40, 0, 0), dev.p(ws_v), dev.p(ws_i),
                                     dev.p(toks), dev.p(c), None))
        res.append((dev.get(logits), int(dev.get(toks)[0]), dev.get(dx)))
    (la, ta, xa), (lb, tb, xb) = res
    assert rel_err(la, lb) < 1e-5
    assert ta == int(np.argmax(la))
    srt = np.sort(lb)
    if srt[-1] - srt[-2] > 1e-4 * np.max(np.abs(lb)):
        assert ta == tb
    assert np.array_equal(xa, E[ta].astype(np.float32))


@pytest.mark.parametrize("fmt", FMTS)
def test_quantize_pack_rounding(vsl, dev, H, fmt):
    """The on-device quantizer: every value within half a step of its block's grid (Q4_0: one step at
    the clamped end of its asymmetric range), the grid's step d from the block's range as documented,
    and the pack's GEMV equal to the GEMV over its dequantized values."""
    rows, K = 300, 256
    w = np.random.default_rng(7).normal(0, 0.02, (rows, K)).astype(np.float16)
    pack = dev.empty((H.vsl_quant_pack_bytes(DT[fmt], rows, K),), np.uint8)
    ok(vsl, H.vsl_quantize_pack(dev.p(dev.put(w)), vsl.VSL_DT_F16, rows, K, DT[fmt], dev.p(pack), None))
    deq = dev.empty((rows, K), np.float32)
    ok(vsl, H.vsl_dequant_pack(dev.p(pack), DT[fmt], rows, K, dev.p(deq), vsl.VSL_DT_F32, None))
    got = dev.get(deq).reshape(-1, 32).astype(np.float64)
    wb = w.astype(np.float64).reshape(-1, 32)
    if fmt == "q8_0":
        step = np.abs(wb).max(axis=1) / 127
        bound = step / 2
    elif fmt == "q4_0":
        wmax = wb[np.arange(len(wb)), np.argmax(np.abs(wb), axis=1)]
        step = np.abs(wmax) / 8
        bound = step
    else:
        step = (wb.max(axis=1) - wb.min(axis=1)) / 15
        bound = step / 2
    err = np.abs(got - wb)
    assert np.all(err <= bound[:, None] * (1 + 1e-5) + 1e-12)
    x = np.random.default_rng(8).normal(0, 1, K).astype(np.float32)
    y = dev.empty((rows,), np.float32)
    ok(vsl, H.vsl_gemv(dev.p(pack), DT[fmt], rows, K, dev.p(dev.put(x)), vsl.VSL_DT_F32, 1, dev.p(y), vsl.VSL_DT_F32,
                       None))
    assert rel_err(dev.get(y), got.reshape(rows, K) @ x.astype(np.float64)) < 1e-5


def test_quant_pack_rejections(vsl, dev, H):
    """K not a multiple of 32, a misaligned pack, blocks past the pack's rows and a float source
    format are refused before any launch."""
    buf = dev.empty((1 << 16,), np.uint8)
    p = dev.p(buf)
    assert H.vsl_quant_pack(p, WF["q8_0"], 0, 4, p + 8192, 4, 48, 0, None) == vsl.VSL_E_INVALID      # K % 32
    assert H.vsl_quant_pack(p, WF["q8_0"], 0, 4, p + 8192 + 16, 4, 32, 0, None) == vsl.VSL_E_INVALID  # alignment
    assert H.vsl_quant_pack(p, WF["q8_0"], 0, 4, p + 8192, 2, 32, 1, None) == vsl.VSL_E_INVALID      # past rows
    assert H.vsl_quant_pack(p, 1, 0, 4, p + 8192, 4, 32, 0, None) == vsl.VSL_E_UNSUPPORTED            # F16 source
    x = dev.empty((64,), np.float32)
    assert H.vsl_gemv(p + 8192, DT["q8_0"], 4, 48, dev.p(x), vsl.VSL_DT_F32, 1, dev.p(x), vsl.VSL_DT_F32,
                      None) == vsl.VSL_E_INVALID
    assert H.vsl_gemv_residual(p + 16, DT["q4_0"], 4, 64, dev.p(x), dev.p(x), None, None) == vsl.VSL_E_INVALID
