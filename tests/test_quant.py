"""Block-quantized GGUF tensors (Q4_0 / Q4_1 / Q8_0), dequantized on load.

Reference behaviour: GGUFLoaderImpl::dequantize_tensor (vk_symbiote/src/GGUFLoader.cpp:1121-1223)
reached from read_tensor_data (:761-793); ids Q4_0 = 13, Q4_1 = 14, Q8_0 = 17 (GGUFLoader.h:18-73),
sizes from calculate_tensor_data_size (:1085-1119).  Files with ggml's ids (2, 3, 8) use ggml's
published block layout instead (low nibbles hold elements 0..15, high nibbles 16..31).

The oracle's orc_dequant is pinned here by hand-assembled blocks whose expected values are written
out literally, by the int8 code table, by the special cases of the reference's scale helper, and by
an error bound against an independent numpy quantizer.  The product's host reader is then compared
with the oracle bit for bit.  Everything in this file runs on the CPU.
"""
import ctypes
import struct

import numpy as np
import pytest

from test_oracle import build_gguf

REF_IDS = {"q4_0": 13, "q4_1": 14, "q8_0": 17}
GGML_IDS = {"q4_0": 2, "q4_1": 3, "q8_0": 8}
BLOCK_BYTES = {"q4_0": 18, "q4_1": 20, "q8_0": 34}


def h(x):
    """binary16 bits of x (numpy rounding)."""
    return int(np.array([x], dtype=np.float16).view(np.uint16)[0])


def dq(orc, raw, raw_type, convention, n, size=None):
    out = np.full(max(n, 1), np.nan, dtype=np.float32)
    buf = np.frombuffer(raw, dtype=np.uint8).copy() if raw else np.zeros(1, np.uint8)
    r = orc.lib().orc_dequant(orc.ptr(buf), len(raw) if size is None else size, raw_type, convention, n,
                              orc.ptr(out))
    return r, out


def bits(a):
    return np.asarray(a, dtype=np.float32).view(np.uint32)


# ---------------------------------------------------------------------------------------------
# numpy quantizer (independent of the oracle; also used to build fixtures for the product tests)
# ---------------------------------------------------------------------------------------------
def np_quantize(x, fmt, convention):
    """Quantize a 1-D float32 array (length a multiple of 32) into raw block bytes."""
    x = np.asarray(x, dtype=np.float32).reshape(-1, 32)
    out = bytearray()
    for blk in x:
        if fmt == "q8_0":
            d = np.float16(np.abs(blk).max() / 127.0)
            inv = 0.0 if d == 0 else 1.0 / np.float32(d)
            q = np.clip(np.rint(blk * inv), -128, 127).astype(np.int8)
            out += struct.pack("<H", h(d)) + q.tobytes()
            continue
        if fmt == "q4_0":
            amax_i = int(np.argmax(np.abs(blk)))
            d = np.float16(blk[amax_i] / -8.0)
            inv = 0.0 if d == 0 else 1.0 / np.float32(d)
            nib = np.clip(np.floor(blk * inv + 8.5), 0, 15).astype(np.uint8)
            head = struct.pack("<H", h(d))
        else:
            lo, hi = float(blk.min()), float(blk.max())
            d = np.float16((hi - lo) / 15.0)
            m = np.float16(lo)
            inv = 0.0 if d == 0 else 1.0 / np.float32(d)
            nib = np.clip(np.floor((blk - np.float32(m)) * inv + 0.5), 0, 15).astype(np.uint8)
            head = struct.pack("<HH", h(d), h(m))
        if convention == 0:   # reference: byte i = elements 2i (low) and 2i+1 (high)
            packed = nib[0::2] | (nib[1::2] << 4)
        else:                 # ggml: byte j = elements j (low) and j+16 (high)
            packed = nib[:16] | (nib[16:] << 4)
        out += head + packed.astype(np.uint8).tobytes()
    return bytes(out)


# ---------------------------------------------------------------------------------------------
# oracle pins
# ---------------------------------------------------------------------------------------------
RAMP = bytes(i | ((15 - i) << 4) for i in range(16))  # byte i: low nibble i, high nibble 15-i


def test_q4_0_nibble_order_reference_ids(orc):
    r, out = dq(orc, struct.pack("<H", h(0.5)) + RAMP, 13, 0, 32)
    assert r == 32
    expect = [-4.0, 3.5, -3.5, 3.0, -3.0, 2.5, -2.5, 2.0, -2.0, 1.5, -1.5, 1.0, -1.0, 0.5, -0.5, 0.0,
              0.0, -0.5, 0.5, -1.0, 1.0, -1.5, 1.5, -2.0, 2.0, -2.5, 2.5, -3.0, 3.0, -3.5, 3.5, -4.0]
    assert out.tolist() == expect


def test_q4_0_nibble_order_ggml_ids(orc):
    r, out = dq(orc, struct.pack("<H", h(0.5)) + RAMP, 2, 1, 32)
    assert r == 32
    expect = [-4.0, -3.5, -3.0, -2.5, -2.0, -1.5, -1.0, -0.5, 0.0, 0.5, 1.0, 1.5, 2.0, 2.5, 3.0, 3.5,
              3.5, 3.0, 2.5, 2.0, 1.5, 1.0, 0.5, 0.0, -0.5, -1.0, -1.5, -2.0, -2.5, -3.0, -3.5, -4.0]
    assert out.tolist() == expect


def test_q4_1_scale_and_min(orc):
    blk = struct.pack("<HH", h(0.25), h(-1.0)) + RAMP
    r, out = dq(orc, blk, 14, 0, 32)
    assert r == 32
    assert out.tolist() == [-1.0, 2.75, -0.75, 2.5, -0.5, 2.25, -0.25, 2.0, 0.0, 1.75, 0.25, 1.5, 0.5, 1.25,
                            0.75, 1.0, 1.0, 0.75, 1.25, 0.5, 1.5, 0.25, 1.75, 0.0, 2.0, -0.25, 2.25, -0.5,
                            2.5, -0.75, 2.75, -1.0]
    r, out = dq(orc, blk, 3, 1, 32)
    assert r == 32
    assert out.tolist() == [-1.0, -0.75, -0.5, -0.25, 0.0, 0.25, 0.5, 0.75, 1.0, 1.25, 1.5, 1.75, 2.0, 2.25,
                            2.5, 2.75, 2.75, 2.5, 2.25, 2.0, 1.75, 1.5, 1.25, 1.0, 0.75, 0.5, 0.25, 0.0,
                            -0.25, -0.5, -0.75, -1.0]


@pytest.mark.parametrize("raw_type,conv", [(17, 0), (8, 1)])
def test_q8_0_every_code_is_signed(orc, raw_type, conv):
    # eight blocks, scale 1.0, codes 0..255 in byte order: a code >= 128 is negative (int8)
    codes = bytes(range(256))
    raw = b"".join(struct.pack("<H", h(1.0)) + codes[32 * b:32 * b + 32] for b in range(8))
    r, out = dq(orc, raw, raw_type, conv, 256)
    assert r == 256
    assert out.tolist() == [float(c) for c in range(128)] + [float(c) for c in range(-128, 0)]
    r, out = dq(orc, struct.pack("<H", h(0.125)) + bytes([0x80, 0x81, 0xFF, 0, 1, 2, 0x7F]) + b"\0" * 25,
                raw_type, conv, 7)
    assert r == 7 and out[:7].tolist() == [-16.0, -15.875, -0.125, 0.0, 0.125, 0.25, 15.875]


def test_reference_scale_helper_special_cases(orc):
    # GGUFLoader.cpp:1137-1138: a subnormal scale is ldexp(mantissa, -24) with the sign dropped and
    # a zero scale is +0; ggml ids use plain binary16 (-2^-24 and -0 keep their sign)
    q = bytes([1, 0xFF]) + b"\0" * 30  # codes +1 and -1
    tiny = 2.0 ** -24
    r, out = dq(orc, struct.pack("<H", 0x8001) + q, 17, 0, 2)
    assert r == 2 and out[:2].tolist() == [tiny, -tiny]
    r, out = dq(orc, struct.pack("<H", 0x8001) + q, 8, 1, 2)
    assert r == 2 and out[:2].tolist() == [-tiny, tiny]
    r, out = dq(orc, struct.pack("<H", 0x83FF) + q, 17, 0, 1)
    assert out[0] == 1023 * tiny
    r, out = dq(orc, struct.pack("<H", 0x8000) + q, 17, 0, 2)  # -0 -> +0: +1*0 = +0, -1*0 = -0
    assert bits(out[:2]).tolist() == [0x00000000, 0x80000000]
    r, out = dq(orc, struct.pack("<H", 0x8000) + q, 8, 1, 2)   # -0 kept: +1*-0 = -0, -1*-0 = +0
    assert bits(out[:2]).tolist() == [0x80000000, 0x00000000]
    r, out = dq(orc, struct.pack("<H", 0xFC00) + q, 17, 0, 2)  # -inf keeps its sign
    assert out[0] == -np.inf and out[1] == np.inf
    r, out = dq(orc, struct.pack("<H", 0xC000) + q, 17, 0, 2)  # normal scales are exact binary16
    assert out[:2].tolist() == [-2.0, 2.0]


def test_partial_and_truncated_blocks(orc):
    raw = struct.pack("<H", h(1.0)) + RAMP + struct.pack("<H", h(2.0)) + RAMP
    r, out = dq(orc, raw, 13, 0, 40)                    # 40 elements: the second block is partial
    assert r == 40
    assert out[32:40].tolist() == [-16.0, 14.0, -14.0, 12.0, -12.0, 10.0, -10.0, 8.0]
    r, out = dq(orc, raw, 13, 0, 64, size=18 + 10)      # the guard stops before a cut block
    assert r == 32
    r, out = dq(orc, raw, 13, 0, 64, size=17)
    assert r == 0


@pytest.mark.parametrize("raw_type,conv", [(15, 0), (16, 0), (18, 0), (6, 1), (7, 1), (12, 1), (13, 1)])
def test_other_block_types_are_rejected(orc, raw_type, conv):
    assert dq(orc, b"\0" * 64, raw_type, conv, 32)[0] == -20


@pytest.mark.parametrize("fmt", ["q4_0", "q4_1", "q8_0"])
@pytest.mark.parametrize("conv", [0, 1])
def test_quantize_dequantize_error_bound(orc, fmt, conv):
    rng = np.random.default_rng(5)
    x = (rng.standard_normal(32 * 64) * 0.02).astype(np.float32)
    x[:32] = 0.0                       # an all-zero block (scale 0)
    x[32:64] = np.linspace(-1, 3, 32)  # a wide, asymmetric block
    raw = np_quantize(x, fmt, conv)
    assert len(raw) == 64 * BLOCK_BYTES[fmt]
    rt = (REF_IDS if conv == 0 else GGML_IDS)[fmt]
    r, out = dq(orc, raw, rt, conv, x.size)
    assert r == x.size
    xb, ob = x.reshape(-1, 32), out.reshape(-1, 32)
    for b in range(xb.shape[0]):
        lo, hi = float(xb[b].min()), float(xb[b].max())
        amax = max(abs(lo), abs(hi))
        if fmt == "q8_0":
            bound = amax / 127.0 * 0.5 * 1.001
        elif fmt == "q4_0":
            bound = amax / 8.0 * 1.001          # the code opposite the extreme may clip by one step
        else:
            bound = (hi - lo) / 15.0 * 0.5 * 1.01 + 2.0 ** -10 * (abs(lo) + abs(hi))
        err = np.abs(xb[b] - ob[b]).max()
        assert err <= bound + 1e-12, (fmt, conv, b, err, bound)
    assert np.all(out[:32] == 0.0)


# ---------------------------------------------------------------------------------------------
# GGUF files: sizes, read_tensor_data, model load
# ---------------------------------------------------------------------------------------------
def _quant_file(tmp_path, conv, n_elem=40):
    """One tensor of each block type, n_elem elements (ref) / 64 (ggml, whole rows of blocks)."""
    rng = np.random.default_rng(9)
    tensors, expect = [], {}
    for fmt in ("q4_0", "q4_1", "q8_0"):
        n = n_elem if conv == 0 else 64
        x = (rng.standard_normal((n + 31) // 32 * 32) * 0.1).astype(np.float32)
        raw = np_quantize(x, fmt, conv)
        rt = (REF_IDS if conv == 0 else GGML_IDS)[fmt]
        tensors.append((f"t.{fmt}", [n], rt, raw))
        expect[fmt] = (rt, raw, n)
    kvs = [("general.alignment", 4, struct.pack("<I", 32))] if conv == 1 else []
    data, start, offs = build_gguf(tensors, kvs, convention="reference" if conv == 0 else "ggml")
    p = tmp_path / f"quant_{conv}.gguf"
    p.write_bytes(data)
    return p, start, offs, expect


@pytest.mark.parametrize("conv", [0, 1])
def test_oracle_reads_quantized_tensors(orc, tmp_path, conv):
    L = orc.lib()
    p, start, offs, expect = _quant_file(tmp_path, conv)
    h_ = ctypes.c_void_p()
    assert L.orc_gguf_open(str(p).encode(), ctypes.byref(h_)) == 0
    try:
        for i, (fmt, (rt, raw, n)) in enumerate(expect.items()):
            idx = L.orc_gguf_find(h_, f"t.{fmt}".encode())
            ds = ctypes.c_uint64()
            L.orc_gguf_tensor_info(h_, idx, None, 0, None, None, None, None, ctypes.byref(ds))
            # calculate_tensor_data_size (:1111-1116): whole blocks, a partial one rounded up
            assert ds.value == len(raw) == (n + 31) // 32 * BLOCK_BYTES[fmt]
            out = np.zeros(64, dtype=np.float32)
            assert L.orc_gguf_read_f32(h_, f"t.{fmt}".encode(), orc.ptr(out), 64) == n
            r, ref = dq(orc, raw, rt, conv, n)
            assert bits(out[:n]).tolist() == bits(ref[:n]).tolist()
    finally:
        L.orc_gguf_close(h_)


# ---------------------------------------------------------------------------------------------
# the product's host reader (GGUFLoader::read_tensor_data) against the oracle, bit for bit
# ---------------------------------------------------------------------------------------------
@pytest.mark.parametrize("conv", [0, 1])
def test_product_reader_dequantizes_like_oracle(vsl, orc, tmp_path, conv):
    L = vsl.engine_lib()
    p, start, offs, expect = _quant_file(tmp_path, conv)
    g = ctypes.c_void_p()
    assert L.vsl_gguf_open(str(p).encode(), ctypes.byref(g)) == 0
    try:
        for fmt, (rt, raw, n) in expect.items():
            out = np.zeros(64, dtype=np.float32)
            assert L.vsl_gguf_read_f32(g, f"t.{fmt}".encode(), out.ctypes.data_as(ctypes.c_void_p), 64) == n
            r, ref = dq(orc, raw, rt, conv, n)
            assert bits(out[:n]).tolist() == bits(ref[:n]).tolist(), fmt
    finally:
        L.vsl_gguf_close(g)


def test_product_reader_scale_helper_and_rejections(vsl, orc, tmp_path):
    L = vsl.engine_lib()
    q = bytes([1, 0xFF, 0x80, 0x7F]) + b"\0" * 28
    tensors = [("neg_sub", [32], 17, struct.pack("<H", 0x8001) + q),
               ("neg_zero", [32], 17, struct.pack("<H", 0x8000) + q),
               ("q5_0", [32], 15, b"\0" * 22)]
    data, _, _ = build_gguf(tensors, [])
    p = tmp_path / "s.gguf"
    p.write_bytes(data)
    g = ctypes.c_void_p()
    assert L.vsl_gguf_open(str(p).encode(), ctypes.byref(g)) == 0
    try:
        for name, (_, _, rt, raw) in zip([b"neg_sub", b"neg_zero"], tensors[:2]):
            out = np.zeros(32, dtype=np.float32)
            assert L.vsl_gguf_read_f32(g, name, out.ctypes.data_as(ctypes.c_void_p), 32) == 32
            r, ref = dq(orc, raw, rt, 0, 32)
            assert bits(out).tolist() == bits(ref).tolist()
        out = np.zeros(32, dtype=np.float32)
        assert L.vsl_gguf_read_f32(g, b"q5_0", out.ctypes.data_as(ctypes.c_void_p), 32) == -20
    finally:
        L.vsl_gguf_close(g)


# ---------------------------------------------------------------------------------------------
# synthetic quantized models written by the product's GGUF writer
# ---------------------------------------------------------------------------------------------
# a tiny Llama-style config whose row lengths (d = 256, F = 768) are whole 32-element blocks
QTINY = dict(hidden_size=256, num_layers=2, num_heads=4, num_kv_heads=2, intermediate_size=768, vocab_size=2048,
             max_position_embeddings=512, rope_theta=10000.0, rms_eps=1e-5)
FMT_CODE = {"q4_0": 2, "q4_1": 3, "q8_0": 4}


@pytest.mark.parametrize("fmt", ["q4_0", "q4_1", "q8_0"])
@pytest.mark.parametrize("convention", ["reference", "ggml"])
def test_synthetic_quantized_gguf(vsl, orc, tmp_path, fmt, convention):
    conv = 0 if convention == "reference" else 1
    p = tmp_path / f"q_{fmt}_{convention}.gguf"
    vsl.write_synthetic_gguf(p, dict(QTINY, dtype=FMT_CODE[fmt]), seed=3, convention=convention)
    L, E = orc.lib(), vsl.engine_lib()
    h_, g = ctypes.c_void_p(), ctypes.c_void_p()
    assert L.orc_gguf_open(str(p).encode(), ctypes.byref(h_)) == 0
    assert E.vsl_gguf_open(str(p).encode(), ctypes.byref(g)) == 0
    try:
        d, F = QTINY["hidden_size"], QTINY["intermediate_size"]
        for name, n in [("token_embd.weight", QTINY["vocab_size"] * d), ("blk.1.ffn_down.weight", d * F),
                        ("blk.0.attn_k.weight", 128 * d), ("blk.0.attn_norm.weight", d)]:
            rt = ctypes.c_uint32()
            idx = L.orc_gguf_find(h_, name.encode())
            L.orc_gguf_tensor_info(h_, idx, None, 0, None, None, ctypes.byref(rt), None, None)
            if name.endswith("norm.weight"):
                assert rt.value == (6 if conv == 0 else 0)  # gains stay F32
            else:
                assert rt.value == (REF_IDS if conv == 0 else GGML_IDS)[fmt]
            a = np.zeros(n, np.float32)
            b = np.zeros(n, np.float32)
            assert L.orc_gguf_read_f32(h_, name.encode(), orc.ptr(a), n) == n
            assert E.vsl_gguf_read_f32(g, name.encode(), b.ctypes.data_as(ctypes.c_void_p), n) == n
            assert bits(a).tolist() == bits(b).tolist()
            if not name.endswith("norm.weight"):
                # within one quantization step of the fp32 draws the blocks were made from
                x = vsl.synthetic_fill_host(n, 0, 3, name)
                step = {"q8_0": 1 / 127, "q4_0": 1 / 8, "q4_1": 1 / 15}[fmt]
                amax = np.abs(x.reshape(-1, 32)).max(1, keepdims=True)
                err = np.abs((a - x).reshape(-1, 32))
                assert np.all(err <= 2.0 * step * amax + 1e-7)
    finally:
        L.orc_gguf_close(h_)
        E.vsl_gguf_close(g)
    m = orc.Model(p)  # dequant-on-load in the oracle model
    assert m.config["hidden_size"] == 256
    m.close()
