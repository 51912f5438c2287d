"""CPU tests of the product's host side: the C ABI exports, GGUF reader/writer, ConfigManager and the
synthetic generators.  No kernel is launched."""
import ctypes
import os
import re
import struct
import subprocess

import numpy as np
import pytest

import vsl_testlib
from test_oracle import build_gguf, _gstr

ROOT = vsl_testlib.ROOT


def _declared(header):
    src = open(os.path.join(ROOT, "include", header)).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    names = re.findall(r"^\s*(?:const\s+)?[A-Za-z_][A-Za-z0-9_]*\s*\**\s*(vsl_[A-Za-z0-9_]+)\s*\(", src, flags=re.M)
    return sorted(set(names))


def _exports(lib):
    out = subprocess.run(["nm", "-D", "--defined-only", lib], capture_output=True, text=True, check=True).stdout
    return {l.split()[-1] for l in out.splitlines() if " T " in l}


def test_c_abi_exports_every_declared_symbol(vsl):
    hip_syms = _exports(vsl.HIP_LIB)
    eng_syms = _exports(vsl.ENGINE_LIB)
    decl_hip, decl_eng = _declared("vsl_hip.h"), _declared("vsl_engine.h")
    assert len(decl_hip) > 40 and len(decl_eng) > 20
    assert not [n for n in decl_hip if n not in hip_syms]
    assert not [n for n in decl_eng if n not in eng_syms]
    # the Python binding declares argtypes for every exported entry point
    vsl.hip()
    vsl.engine_lib()
    assert set(decl_hip) <= set(vsl._HIP_SIGS) and set(decl_eng) <= set(vsl._ENGINE_SIGS)


def test_header_constants_match_the_binding(vsl):
    """The Python binding's copies of the header's enum values (status codes, sampler modes, the
    seeded top-k limit) equal the header's."""
    src = re.sub(r"/\*.*?\*/", "", open(os.path.join(ROOT, "include", "vsl_hip.h")).read(), flags=re.S)
    val = {n: int(v) for n, v in re.findall(r"\b(VSL_[A-Z0-9_]+)\s*=\s*(-?\d+)", src)}
    assert val["VSL_MAX_TOP_K"] == vsl.MAX_TOP_K
    assert (val["VSL_E_INVALID"], val["VSL_E_UNSUPPORTED"], val["VSL_E_CAPACITY"]) == (
        vsl.VSL_E_INVALID, vsl.VSL_E_UNSUPPORTED, vsl.VSL_E_CAPACITY)
    assert (val["VSL_SAMPLE_GREEDY"], val["VSL_SAMPLE_REFERENCE"], val["VSL_SAMPLE_TOPK_SEEDED"]) == (
        vsl.SAMPLE_GREEDY, vsl.SAMPLE_REFERENCE, vsl.SAMPLE_TOPK_SEEDED)


def test_gemm_direct_query(vsl):
    """vsl_gemm_f16_direct (host arithmetic only): whole 256 x 256 or 128 x 256 tiles covering >= 192
    CUs, or a K split reaching 192 items, count as direct-to-LDS; a 128-row SwiGLU (64 tiles, no K split
    for SwiGLU) does not; widths off the 256 / 128 grid never do."""
    H = vsl.hip()
    SW, F32, RES = 3, 0, 2
    assert H.vsl_gemm_f16_direct(512, 14336, 4096, SW) == 1      # 8B gate/up, 2 x 112 tiles
    assert H.vsl_gemm_f16_direct(128, 8192, 2048, SW) == 0       # 1B gate/up of a 128-row prompt
    assert H.vsl_gemm_f16_direct(512, 8192, 2048, SW) == 1       # 1B gate/up of a 512-row chunk
    assert H.vsl_gemm_f16_direct(512, 4096, 14336, RES) == 1     # 8B down: K split
    assert H.vsl_gemm_f16_direct(128, 2048, 8192, RES | 0x400) == 1  # flags beyond the epilogue ignored
    assert H.vsl_gemm_f16_direct(512, 4000, 4096, F32) == 0      # N off the tile grid
    assert H.vsl_gemm_f16_direct(512, 4096, 4000, F32) == 0      # K not a multiple of 128


def test_no_cpu_fallback_in_the_product(vsl):
    """The product libraries link HIP and nothing from the oracle."""
    for lib in (vsl.HIP_LIB, vsl.ENGINE_LIB):
        out = subprocess.run(["nm", "-D", lib], capture_output=True, text=True, check=True).stdout
        assert "orc_" not in out
    deps = subprocess.run(["ldd", vsl.ENGINE_LIB], capture_output=True, text=True).stdout
    assert "libvsl_oracle" not in deps and "libvsl_hip" in deps


def _gguf(vsl, path):
    L = vsl.engine_lib()
    h = ctypes.c_void_p()
    rc = L.vsl_gguf_open(str(path).encode(), ctypes.byref(h))
    return rc, h


def test_product_gguf_reader_matches_hand_layout(vsl, tmp_path):
    L = vsl.engine_lib()
    a = np.arange(12, dtype=np.float32) * 0.25
    b = (np.arange(6, dtype=np.float32) - 1.5).astype(np.float16)
    kvs = [("llama.embedding_length", 4, struct.pack("<I", 128)), ("llama.attention.head_count", 4, struct.pack("<I", 2)),
           ("llama.rope.freq_base", 6, struct.pack("<f", 10000.0)), ("general.architecture", 8, _gstr("llama"))]
    data, start, offs = build_gguf([("t.a", [4, 3], 6, a.tobytes()), ("t.b", [6], 48, b.tobytes())], kvs)
    p = tmp_path / "r.gguf"
    p.write_bytes(data)
    rc, h = _gguf(vsl, p)
    assert rc == 0
    try:
        tc, mc, ds = ctypes.c_uint64(), ctypes.c_uint64(), ctypes.c_uint64()
        ver, conv = ctypes.c_uint32(), ctypes.c_int()
        L.vsl_gguf_info(h, ctypes.byref(tc), ctypes.byref(mc), ctypes.byref(ver), ctypes.byref(conv), ctypes.byref(ds))
        assert (tc.value, mc.value, ver.value, conv.value, ds.value) == (2, 4, 3, 0, start)
        out = np.zeros(16, np.float32)
        assert L.vsl_gguf_read_f32(h, b"t.a", out.ctypes.data_as(ctypes.c_void_p), 16) == 12
        assert np.array_equal(out[:12], a)
        assert L.vsl_gguf_read_f32(h, b"t.b", out.ctypes.data_as(ctypes.c_void_p), 16) == 6
        assert np.array_equal(out[:6], b.astype(np.float32))
        off, size, rt, nd = ctypes.c_uint64(), ctypes.c_uint64(), ctypes.c_uint32(), ctypes.c_uint32()
        dims = (ctypes.c_uint64 * 4)()
        assert L.vsl_gguf_tensor(h, b"t.a", ctypes.byref(off), ctypes.byref(size), ctypes.byref(rt), ctypes.byref(nd), dims) == 0
        assert (off.value, size.value, rt.value, nd.value, dims[0], dims[1]) == (start + offs[0], 48, 6, 2, 4, 3)
        assert L.vsl_gguf_tensor(h, b"zzz", None, None, None, None, None) == -30
        spec = vsl.ModelSpec()
        L.vsl_gguf_model_config(h, ctypes.byref(spec))
        assert spec.hidden_size == 128 and spec.num_heads == 2 and spec.num_kv_heads == 2 and spec.head_dim == 64
        assert spec.num_layers == 32 and spec.vocab_size == 32000  # ModelConfig defaults (Common.h:56-76)
    finally:
        L.vsl_gguf_close(h)


def test_product_gguf_error_codes(vsl, tmp_path):
    assert _gguf(vsl, tmp_path / "missing.gguf")[0] == -1
    bad = tmp_path / "bad.gguf"
    bad.write_bytes(b"GGML" + b"\0" * 40)
    assert _gguf(vsl, bad)[0] == -2
    data, _, _ = build_gguf([("t", [4], 6, b"\0" * 16)], [("k", 8, _gstr("value"))])
    tm = tmp_path / "tm.gguf"
    tm.write_bytes(data[:24 + 8 + 1 + 4 + 3])
    assert _gguf(vsl, tm)[0] == -3
    hdr = 24 + len(_gstr("k")) + 4 + len(_gstr("value"))
    ti = tmp_path / "ti.gguf"
    ti.write_bytes(data[:hdr + 10])
    assert _gguf(vsl, ti)[0] == -4
    q = tmp_path / "q.gguf"
    q.write_bytes(build_gguf([("t", [32], 15, b"\0" * 22)], [])[0])  # Q5_0: dequantize_tensor's -20
    rc, h = _gguf(vsl, q)
    assert rc == 0
    out = np.zeros(64, np.float32)
    assert vsl.engine_lib().vsl_gguf_read_f32(h, b"t", out.ctypes.data_as(ctypes.c_void_p), 64) == -20
    vsl.engine_lib().vsl_gguf_close(h)


def _one_tensor_gguf(dims, raw_type, offset, payload):
    """A reference-convention file with one tensor "t" whose offset field is given literally."""
    out = bytearray(struct.pack("<IIQQ", 0x46554747, 3, 1, 0))
    out += _gstr("t") + struct.pack("<I", len(dims)) + b"".join(struct.pack("<Q", d) for d in dims)
    out += struct.pack("<IQ", raw_type, offset)
    start = len(out)
    return bytes(out + payload), start


def test_product_gguf_rejects_out_of_range_tensors(vsl, tmp_path):
    """Tensor infos of an untrusted file that point outside it: an offset that puts the tensor's start
    just below 2^64 (so that start + size wraps to a small number) and a size past the end of the file
    read as -11 (no pointer outside the mapping is formed); a dimension product that overflows 64 bits,
    or whose byte size would, is a tensor-info error (-4) at load."""
    L = vsl.engine_lib()
    out = np.zeros(64, np.float32)
    # start + offset = 2^64 - 64; 32 F32 elements = 128 bytes, so start + offset + size wraps to 64
    _, start = _one_tensor_gguf([32], 6, 0, b"")
    data, _ = _one_tensor_gguf([32], 6, 2**64 - 64 - start, b"\0" * 256)
    p = tmp_path / "wrap.gguf"
    p.write_bytes(data)
    rc, h = _gguf(vsl, p)
    assert rc == 0
    assert L.vsl_gguf_read_f32(h, b"t", out.ctypes.data_as(ctypes.c_void_p), 64) == -11
    L.vsl_gguf_close(h)
    # the tensor's bytes run past the end of the file by one byte
    data, _ = _one_tensor_gguf([16], 6, 0, b"\0" * 63)
    p = tmp_path / "short.gguf"
    p.write_bytes(data)
    rc, h = _gguf(vsl, p)
    assert rc == 0
    assert L.vsl_gguf_read_f32(h, b"t", out.ctypes.data_as(ctypes.c_void_p), 64) == -11
    L.vsl_gguf_close(h)
    # the same tensor with every byte present reads
    data, _ = _one_tensor_gguf([16], 6, 0, np.arange(16, dtype=np.float32).tobytes())
    p = tmp_path / "ok.gguf"
    p.write_bytes(data)
    rc, h = _gguf(vsl, p)
    assert rc == 0
    assert L.vsl_gguf_read_f32(h, b"t", out.ctypes.data_as(ctypes.c_void_p), 64) == 16
    assert np.array_equal(out[:16], np.arange(16, dtype=np.float32))
    L.vsl_gguf_close(h)
    # 2^32 * 2^32 * 2 elements wrap to 0; 2^62 F32 elements are 2^64 bytes
    for dims in ([2**32, 2**32, 2], [2**62]):
        data, _ = _one_tensor_gguf(dims, 6, 0, b"\0" * 64)
        p = tmp_path / "dims.gguf"
        p.write_bytes(data)
        assert _gguf(vsl, p)[0] == -4


@pytest.mark.parametrize("convention", ["reference", "ggml"])
@pytest.mark.parametrize("dtype", [0, 1])
def test_writer_roundtrip_through_both_readers(vsl, orc, tmp_path, convention, dtype):
    cfg = dict(hidden_size=128, num_layers=2, num_heads=2, num_kv_heads=1, intermediate_size=256, vocab_size=300,
               max_position_embeddings=64, rope_theta=10000.0, rms_eps=1e-5, dtype=dtype)
    p = tmp_path / f"m_{convention}_{dtype}.gguf"
    vsl.write_synthetic_gguf(p, cfg, seed=11, convention=convention)
    m = orc.Model(p)
    c = m.config
    assert (c["hidden_size"], c["num_layers"], c["num_heads"], c["num_kv_heads"], c["intermediate_size"],
            c["vocab_size"], c["head_dim"]) == (128, 2, 2, 1, 256, 300, 64)
    # the data section starts 32-aligned under both the reference's rule and ggml's
    L = orc.lib()
    h = ctypes.c_void_p()
    assert L.orc_gguf_open(str(p).encode(), ctypes.byref(h)) == 0
    assert L.orc_gguf_data_start(h) % 32 == 0
    assert L.orc_gguf_convention(h) == (1 if convention == "ggml" else 0)
    L.orc_gguf_close(h)
    # every tensor reads identically through the product loader and the oracle's reader
    rc, g = _gguf(vsl, p)
    assert rc == 0
    names = ["token_embd.weight", "output.weight", "output_norm.weight", "blk.1.attn_k.weight", "blk.0.ffn_down.weight",
             "blk.0.attn_norm.weight"]
    for n in names:
        a = np.zeros(300 * 128, np.float32)
        b = np.zeros(300 * 128, np.float32)
        na = vsl.engine_lib().vsl_gguf_read_f32(g, n.encode(), a.ctypes.data_as(ctypes.c_void_p), a.size)
        hh = ctypes.c_void_p()
        L.orc_gguf_open(str(p).encode(), ctypes.byref(hh))
        nb = L.orc_gguf_read_f32(hh, n.encode(), orc.ptr(b), b.size)
        L.orc_gguf_close(hh)
        assert na == nb > 0 and np.array_equal(a[:na], b[:nb])
    vsl.engine_lib().vsl_gguf_close(g)
    # linear weights follow the synthetic generator
    w = np.zeros(128 * 64, np.float32)
    hh = ctypes.c_void_p()
    L.orc_gguf_open(str(p).encode(), ctypes.byref(hh))
    L.orc_gguf_read_f32(hh, b"blk.1.attn_k.weight", orc.ptr(w), w.size)
    L.orc_gguf_close(hh)
    expect = orc.fill_normal(w.size, orc.F16 if dtype == 1 else orc.F32, 11, "blk.1.attn_k.weight").astype(np.float32)
    assert np.array_equal(w, expect)


def test_host_generator_matches_oracle_generator(vsl, orc):
    for dt in (vsl.VSL_DT_F32, vsl.VSL_DT_F16):
        a = vsl.synthetic_fill_host(300001, dt, 5, "blk.3.ffn_up.weight", 0.0, 0.02)
        b = orc.fill_normal(300001, dt, 5, "blk.3.ffn_up.weight", 0.0, 0.02)
        assert np.array_equal(a.view(np.uint8), b.view(np.uint8))


def test_config_manager_args_and_toml(vsl, tmp_path):
    L = vsl.engine_lib()
    L.vsl_config_reset()
    args = [b"prog", b"--model", b"m.gguf", b"--vram-gb", b"200", b"--disable-gpu", b"--device", b"0",
            b"--seed", b"42", b"--kv-capacity", b"32768"]
    arr = (ctypes.c_char_p * len(args))(*args)
    assert L.vsl_config_load_args(len(args), arr) == 0
    eg, dev, kv, seed, vram = ctypes.c_int(), ctypes.c_int(), ctypes.c_uint32(), ctypes.c_uint64(), ctypes.c_float()
    L.vsl_config_get(ctypes.byref(eg), ctypes.byref(dev), ctypes.byref(kv), ctypes.byref(seed), ctypes.byref(vram))
    assert (eg.value, dev.value, kv.value, seed.value, vram.value) == (0, 0, 32768, 42, 200.0)
    # an engine refuses to open with the GPU disabled: this backend has no CPU path
    eng = ctypes.c_void_p()
    spec = vsl.make_spec(vsl.TINY)
    rc = L.vsl_engine_open_synthetic(ctypes.byref(spec), 0, None, ctypes.byref(eng))
    assert rc != 0 and b"GPU disabled" in L.vsl_engine_last_error()
    # TOML subset: sections, comments, floats accepted for the budgets
    t = tmp_path / "c.toml"
    t.write_text("# comment\n[memory]\nvram_budget_gb = 8.5\nram_budget_gb = 64\n[performance]\n"
                 "enable_gpu = true\nkv_capacity = 4096 # trailing\n[model]\npath = \"x.gguf\"\n")
    L.vsl_config_reset()
    assert L.vsl_config_load_file(str(t).encode()) == 0
    L.vsl_config_get(ctypes.byref(eg), ctypes.byref(dev), ctypes.byref(kv), ctypes.byref(seed), ctypes.byref(vram))
    assert (eg.value, kv.value, vram.value) == (1, 4096, 8.5)
    out = tmp_path / "saved.toml"
    assert L.vsl_config_save_file(str(out).encode()) == 0
    L.vsl_config_reset()
    assert L.vsl_config_load_file(str(out).encode()) == 0
    L.vsl_config_get(ctypes.byref(eg), ctypes.byref(dev), ctypes.byref(kv), ctypes.byref(seed), ctypes.byref(vram))
    assert (eg.value, kv.value, vram.value) == (1, 4096, 8.5)
    t2 = tmp_path / "bad.toml"
    t2.write_text("[memory]\nvram_budget_gb = 1000\n")
    assert L.vsl_config_load_file(str(t2).encode()) != 0  # validate_config: VRAM above 288 GB
    L.vsl_config_reset()


def _gguf_packs(vsl, path):
    L = vsl.engine_lib()
    g = ctypes.c_void_p()
    assert L.vsl_gguf_open(str(path).encode(), ctypes.byref(g)) == 0
    try:
        n = ctypes.c_uint64()
        assert L.vsl_gguf_pack_count(g, ctypes.byref(n)) == 0
        out = {}
        for i in range(n.value):
            info, name = vsl.PackInfo(), ctypes.create_string_buffer(256)
            assert L.vsl_gguf_pack(g, i, ctypes.byref(info), name, 256) == 0
            out[name.value.decode()] = info
        assert L.vsl_gguf_pack(g, n.value, ctypes.byref(vsl.PackInfo()), None, 0) == -30
        return out
    finally:
        L.vsl_gguf_close(g)


# name -> (PackType, layer, priority), by the reference's rules (GGUFLoader.cpp:1264-1315): type by
# substring in a fixed order (ffn_up files under the gate type; only attn_norm / ffn_norm are norms,
# so output_norm is HEAD); layer = the first "blk.<digits>" anywhere; priority 0.5, +0.2 "attn",
# +0.3 "token_embd"/"output", +0.1 layer < 4, capped at 1.0
PACK_RULES = {
    "token_embd.weight": (10, 0, 0.9), "output.weight": (11, 0, 0.9), "output_norm.weight": (11, 0, 0.9),
    "blk.0.attn_q.weight": (0, 0, 0.8), "blk.3.attn_k.weight": (1, 3, 0.8), "blk.4.attn_v.weight": (2, 4, 0.7),
    "blk.17.attn_output.weight": (3, 17, 1.0), "blk.2.ffn_gate.weight": (4, 2, 0.6),
    "blk.5.ffn_up.weight": (4, 5, 0.5), "blk.9.ffn_down.weight": (6, 9, 0.5), "blk.1.attn_norm.weight": (7, 1, 0.8),
    "blk.12.ffn_norm.weight": (7, 12, 0.5), "x.blk.y.blk.21.misc": (255, 21, 0.5), "rope_freqs.weight": (255, 0, 0.6),
}


def test_pack_metadata_rules(vsl, tmp_path):
    tensors = [(n, [4 + i], 6, np.arange(4 + i, dtype=np.float32).tobytes()) for i, n in enumerate(PACK_RULES)]
    data, start, offs = build_gguf(tensors, [("llama.embedding_length", 4, struct.pack("<I", 64))])
    p = tmp_path / "packs.gguf"
    p.write_bytes(data)
    packs = _gguf_packs(vsl, p)
    assert set(packs) == set(PACK_RULES)
    ids = set()
    for (name, dims, _, raw), off in zip(tensors, offs):
        info = packs[name]
        t, layer, prio = PACK_RULES[name]
        assert (info.type, info.layer_idx, info.head_idx, info.alignment) == (t, layer, 0, 256), name
        assert abs(info.base_priority - prio) < 1e-6, (name, info.base_priority)
        assert info.compressed_size == info.decompressed_size == len(raw)
        assert info.file_offset == start + off
        assert (info.tier, info.dtype, info.resident_bytes, info.device_ptr) == (-1, -1, 0, None)
        ids.add(info.pack_id)
    assert len(ids) == len(PACK_RULES) and 0 not in ids  # std::hash of distinct names
