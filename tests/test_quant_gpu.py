"""Block-quantized GGUF models on the MI355X: vsl_convert_weights against the oracle's dequantize_tensor
restatement (bit for bit), and the engine opened from Q4_0 / Q4_1 / Q8_0 files against the oracle
model that dequantizes the same file on load."""
import ctypes
import struct

import numpy as np
import pytest

import vsl_testlib
from test_quant import GGML_IDS, QTINY, REF_IDS, FMT_CODE, bits, dq, np_quantize

pytestmark = pytest.mark.gpu

WF = {"q4_0": 2, "q4_1": 3, "q8_0": 4}


def _blocks(fmt, conv, n_blocks, seed):
    """Random blocks from the numpy quantizer, then blocks with the scales the reference's helper
    treats specially (negative subnormal, -0, smallest subnormal) and a large one."""
    rng = np.random.default_rng(seed)
    x = (rng.standard_normal(32 * n_blocks) * 0.05).astype(np.float32)
    raw = bytearray(np_quantize(x, fmt, conv))
    bb = {"q4_0": 18, "q4_1": 20, "q8_0": 34}[fmt]
    for i, sc in enumerate([0x8001, 0x8000, 0x0001, 0x83FF, 0x7BFF, 0x0400]):
        b = (3 + 5 * i) % n_blocks
        raw[b * bb:b * bb + 2] = struct.pack("<H", sc)
        if fmt == "q4_1":  # min: negative subnormal / tiny
            raw[b * bb + 2:b * bb + 4] = struct.pack("<H", 0x8002 if i % 2 else 0x0003)
    return bytes(raw)


@pytest.mark.parametrize("fmt", ["q4_0", "q4_1", "q8_0"])
@pytest.mark.parametrize("conv", [0, 1])
@pytest.mark.parametrize("n", [32 * 2048, 32 * 777 - 5, 40])
def test_convert_weights_bit_exact(vsl, orc, fmt, conv, n):
    """vsl_convert_weights == orc_dequant bit for bit (fp32 output), and == its binary16 rounding
    (fp16 output); partial last blocks; the scale special cases."""
    H = vsl.hip()
    dev = vsl_testlib.Dev()
    nb = (n + 31) // 32
    raw = _blocks(fmt, conv, nb, seed=n)
    rt = (REF_IDS if conv == 0 else GGML_IDS)[fmt]
    r, ref = dq(orc, raw, rt, conv, n)
    assert r == n
    assert H.vsl_weight_bytes(WF[fmt], n) == len(raw)
    src = dev.put(np.frombuffer(raw, np.uint8))
    out32 = dev.empty(n, np.float32)
    out16 = dev.empty(n, np.float16)
    vsl.check(H.vsl_convert_weights(dev.p(src), WF[fmt], conv, n, dev.p(out32), vsl.VSL_DT_F32, None))
    vsl.check(H.vsl_convert_weights(dev.p(src), WF[fmt], conv, n, dev.p(out16), vsl.VSL_DT_F16, None))
    g32 = dev.get(out32)
    g16 = dev.get(out16)
    assert bits(g32).tolist() == bits(ref[:n]).tolist()
    assert np.array_equal(g16.view(np.uint16), ref[:n].astype(np.float16).view(np.uint16))
    dev.release()


def test_convert_weights_float_and_errors(vsl):
    H = vsl.hip()
    dev = vsl_testlib.Dev()
    rng = np.random.default_rng(4)
    x = (rng.standard_normal(10007) * 3).astype(np.float32)
    x[:6] = [0.0, -0.0, 1e-7, -6e-8, 70000.0, 2.0 ** -25 * 3]  # subnormal / overflow / tie cases
    src32 = dev.put(x)
    src16 = dev.put(x.astype(np.float16))
    o16 = dev.empty(x.size, np.float16)
    o32 = dev.empty(x.size, np.float32)
    vsl.check(H.vsl_convert_weights(dev.p(src32), vsl.VSL_WF_F32, 0, x.size, dev.p(o16), vsl.VSL_DT_F16, None))
    vsl.check(H.vsl_convert_weights(dev.p(src16), vsl.VSL_WF_F16, 0, x.size, dev.p(o32), vsl.VSL_DT_F32, None))
    assert np.array_equal(dev.get(o16).view(np.uint16), x.astype(np.float16).view(np.uint16))
    assert np.array_equal(dev.get(o32).view(np.uint32), x.astype(np.float16).astype(np.float32).view(np.uint32))
    # rejected before any launch: unknown format / layout / dtype, misaligned dst, overlap
    assert H.vsl_convert_weights(dev.p(src32), 9, 0, 64, dev.p(o32), 0, None) == -103
    assert H.vsl_convert_weights(dev.p(src32), 0, 5, 64, dev.p(o32), 0, None) == -100
    assert H.vsl_convert_weights(dev.p(src32), 0, 0, 64, dev.p(o32), 2, None) == -103
    assert H.vsl_convert_weights(dev.p(src32), 0, 0, 64, dev.p(o32) + 4, 0, None) == -100
    assert H.vsl_convert_weights(dev.p(src32), 1, 0, 64, dev.p(src32) + 16, 0, None) == -100
    dev.release()


@pytest.fixture(scope="module")
def qfiles(vsl, tmp_path_factory):
    d = tmp_path_factory.mktemp("quant")
    files = {}
    for fmt in ("q4_0", "q4_1", "q8_0"):
        for conv in ("reference", "ggml"):
            p = d / f"{fmt}_{conv}.gguf"
            vsl.write_synthetic_gguf(p, dict(QTINY, dtype=FMT_CODE[fmt]), seed=5, convention=conv)
            files[fmt, conv] = p
    return files


def _prompt(orc):
    return orc.random_ids(24, QTINY["vocab_size"], 2)


@pytest.mark.parametrize("fmt", ["q4_0", "q4_1", "q8_0"])
@pytest.mark.parametrize("conv", ["reference", "ggml"])
def test_quantized_model_fp32_packs(vsl, orc, qfiles, fmt, conv):
    """dequant_f32 packs hold exactly the dequantized values; greedy 32 tokens identical to the oracle
    model that dequantizes the same file, logits within 1e-4 relative (the fp32 tolerance)."""
    p = qfiles[fmt, conv]
    m = orc.Model(p)
    prompt = _prompt(orc)
    ref_toks, ref_lg = m.generate(prompt, 32, logits=True)
    L, E = orc.lib(), None
    h_ = ctypes.c_void_p()
    assert L.orc_gguf_open(str(p).encode(), ctypes.byref(h_)) == 0
    with vsl.Engine(p, kv_capacity=64, dequant_f32=True) as e:
        assert e.config["dtype"] == 0
        for name in ("token_embd.weight", "output.weight", "blk.1.ffn_down.weight", "blk.0.attn_q.weight"):
            n = QTINY["vocab_size"] * 256 if "token" in name or "output" in name else \
                (256 * 768 if "ffn" in name else 256 * 256)
            want = np.zeros(n, np.float32)
            assert L.orc_gguf_read_f32(h_, name.encode(), orc.ptr(want), n) == n
            got = e.read_tensor(name, n * 4)
            assert bits(got).tolist() == bits(want).tolist(), name
        toks, lg = e.generate_ids(prompt, 32, return_logits=True)
    L.orc_gguf_close(h_)
    m.close()
    scale = np.max(np.abs(ref_lg))
    assert np.array_equal(toks, ref_toks)
    assert np.max(np.abs(lg - ref_lg)) < 1e-4 * scale


@pytest.mark.parametrize("fmt,conv", [("q4_0", "reference"), ("q8_0", "ggml"), ("q4_1", "reference")])
def test_quantized_model_fp16_packs(vsl, orc, qfiles, fmt, conv):
    """Default fp16 packs (the decode on them too, quant_decode off): each pack is the binary16 rounding
    of the dequantized values; the forward pass over those packs (MFMA prefill, fp16 KV cache) matches
    the oracle over the same resident weights: greedy tokens identical, logits within max-abs 2e-2."""
    from test_engine_gpu import _oracle_from_engine
    p = qfiles[fmt, conv]
    prompt = _prompt(orc)
    L = orc.lib()
    h_ = ctypes.c_void_p()
    assert L.orc_gguf_open(str(p).encode(), ctypes.byref(h_)) == 0
    with vsl.Engine(p, kv_capacity=64, quant_decode=False) as e:
        assert e.config["dtype"] == 1
        for name, n in (("token_embd.weight", QTINY["vocab_size"] * 256), ("blk.0.ffn_gate.weight", 256 * 768)):
            want = np.zeros(n, np.float32)
            assert L.orc_gguf_read_f32(h_, name.encode(), orc.ptr(want), n) == n
            got = e.read_tensor(name, n * 2)
            assert np.array_equal(got.view(np.uint16), want.astype(np.float16).view(np.uint16)), name
        toks, lg = e.generate_ids(prompt, 32, return_logits=True)
        m = _oracle_from_engine(orc, e, dict(QTINY, dtype=1))
    L.orc_gguf_close(h_)
    ref_toks, ref_lg = m.generate(prompt, 32, kv_f16=True, logits=True)
    m.close()
    assert np.max(np.abs(lg - ref_lg)) < 2e-2, np.max(np.abs(lg - ref_lg))
    assert np.array_equal(toks, ref_toks)


@pytest.mark.parametrize("fmt", ["q4_0", "q4_1", "q8_0"])
@pytest.mark.parametrize("conv", ["reference", "ggml"])
def test_quant_decode_against_the_file(vsl, orc, qfiles, fmt, conv):
    """The default engine on a quantized file: the decode GEMVs read the resident blocks (the exact
    dequantized values), the MFMA prompt pass the fp16 packs; against the oracle that dequantizes the
    file (fp32 weights, fp16 KV cache): greedy tokens identical, logits within max-abs 2e-2; and the
    same tokens as the engine with quant_decode off."""
    p = qfiles[fmt, conv]
    prompt = _prompt(orc)
    m = orc.Model(p)
    ref_toks, ref_lg = m.generate(prompt, 32, kv_f16=True, logits=True)
    m.close()
    with vsl.Engine(p, kv_capacity=64) as e:
        toks, lg = e.generate_ids(prompt, 32, return_logits=True)
    with vsl.Engine(p, kv_capacity=64, quant_decode=False) as e:
        toks_off = e.generate_ids(prompt, 32)
    assert np.max(np.abs(lg - ref_lg)) < 2e-2, np.max(np.abs(lg - ref_lg))
    assert np.array_equal(toks, ref_toks)
    assert np.array_equal(toks, toks_off)


@pytest.mark.parametrize("fmt", ["q4_0", "q8_0"])
def test_quant_decode_mixed_operands(vsl, orc, tmp_path, fmt):
    """A reference-layout file whose FFN width (712) is a multiple of 8 but not of 32: blocks straddle
    the rows of ffn_down, so the down projection decodes from its expanded pack while the QKV, O and
    gate/up GEMVs read resident blocks (and the prompt runs token by token: FFN is not a multiple of
    64). Against the oracle that dequantizes the file: greedy tokens identical, logits within max-abs
    2e-2, and the same tokens as with quant_decode off."""
    cfg = dict(QTINY, intermediate_size=712, dtype=FMT_CODE[fmt])
    p = tmp_path / f"mixed_{fmt}.gguf"
    vsl.write_synthetic_gguf(p, cfg, seed=9, convention="reference")
    prompt = _prompt(orc)
    m = orc.Model(p)
    ref_toks, ref_lg = m.generate(prompt, 24, kv_f16=True, logits=True)
    m.close()
    with vsl.Engine(p, kv_capacity=64) as e:
        toks, lg = e.generate_ids(prompt, 24, return_logits=True)
        wb_on = e.weight_bytes()
    with vsl.Engine(p, kv_capacity=64, quant_decode=False) as e:
        toks_off = e.generate_ids(prompt, 24)
        wb_off = e.weight_bytes()
    # the block packs held: [Wq;Wk;Wv], Wo and [Wgate;Wup] of every layer and W_out, not Wdown
    H = vsl.hip()
    d, F, V, L = cfg["hidden_size"], cfg["intermediate_size"], cfg["vocab_size"], cfg["num_layers"]
    hd = d // cfg["num_heads"]
    dt = {"q4_0": vsl.VSL_DT_Q4_0, "q8_0": vsl.VSL_DT_Q8_0}[fmt]
    per_layer = (H.vsl_quant_pack_bytes(dt, (cfg["num_heads"] + 2 * cfg["num_kv_heads"]) * hd, d)
                 + H.vsl_quant_pack_bytes(dt, d, cfg["num_heads"] * hd) + H.vsl_quant_pack_bytes(dt, 2 * F, d))
    assert H.vsl_quant_pack_bytes(dt, d, F) == 0  # K % 32 != 0: no pack for the down projection
    assert wb_on - wb_off == L * per_layer + H.vsl_quant_pack_bytes(dt, V, d)
    assert np.max(np.abs(lg - ref_lg)) < 2e-2, np.max(np.abs(lg - ref_lg))
    assert np.array_equal(toks, ref_toks)
    assert np.array_equal(toks, toks_off)


@pytest.mark.parametrize("fmt", ["q4_0", "q4_1", "q8_0"])
def test_synthetic_quantized_engine(vsl, orc, fmt):
    """A synthetic model quantized on the device (vsl_quantize_pack), expanded packs in fp32
    (dequant_f32): those hold exactly the values the decode GEMVs read from the blocks, so the oracle
    over the engine's resident fp32 weights is the same model: greedy 24 tokens identical, logits
    within 1e-4 relative; and the fp16-pack variant (MFMA prompt pass on the fp16-rounded values)
    within max-abs 2e-2 of its own oracle with identical tokens."""
    from test_engine_gpu import _oracle_from_engine
    cfg = dict(QTINY, dtype=FMT_CODE[fmt])
    prompt = _prompt(orc)
    with vsl.Engine(spec=cfg, seed=4, kv_capacity=64, dequant_f32=True) as e:
        assert e.config["dtype"] == 0
        toks, lg = e.generate_ids(prompt, 24, return_logits=True)
        m = _oracle_from_engine(orc, e, dict(cfg, dtype=0))
    ref_toks, ref_lg = m.generate(prompt, 24, logits=True)
    m.close()
    assert np.array_equal(toks, ref_toks)
    assert np.max(np.abs(lg - ref_lg)) < 1e-4 * np.max(np.abs(ref_lg))
    with vsl.Engine(spec=cfg, seed=4, kv_capacity=64) as e:
        assert e.config["dtype"] == 1
        toks16, lg16 = e.generate_ids(prompt, 24, return_logits=True)
        m = _oracle_from_engine(orc, e, dict(cfg, dtype=1))
    ref_toks16, ref_lg16 = m.generate(prompt, 24, kv_f16=True, logits=True)
    m.close()
    assert np.max(np.abs(lg16 - ref_lg16)) < 2e-2
    assert np.array_equal(toks16, ref_toks16)
