"""Pins of the oracle (CPU restatement) against what the mathematics and published vectors fix.

Each test names the reference behaviour it pins.  None of them retypes the oracle's formula: they
use known-answer vectors, closed forms, invariants, library routines (numpy / transformers), or
hand-computed byte layouts.
"""
import ctypes
import math
import struct

import numpy as np
import pytest


# ---------------------------------------------------------------------------------------------
# fp16 <-> fp32 (GGUFLoader.cpp:1225-1262 conversion; binary16 KV cache rounding)
# ---------------------------------------------------------------------------------------------
def test_h2f_exhaustive(orc):
    L = orc.lib()
    bits = np.arange(65536, dtype=np.uint32)
    ours = np.array([L.orc_h2f(int(b)) for b in bits], dtype=np.float32)
    ref = bits.astype(np.uint16).view(np.float16).astype(np.float32)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(ours), nan)
    assert np.array_equal(ours[~nan].view(np.uint32), ref[~nan].view(np.uint32))


def test_f2h_round_to_nearest_even(orc):
    L = orc.lib()
    rng = np.random.default_rng(3)
    # random bit patterns across the whole float range, plus exact half-ulp ties
    pats = rng.integers(0, 2**32, size=200000, dtype=np.uint64).astype(np.uint32)
    vals = pats.view(np.float32)
    vals = vals[np.isfinite(vals)]
    h = np.arange(0, 0x7C00, 7, dtype=np.uint32).astype(np.uint16).view(np.float16).astype(np.float64)
    ties = ((h[:-1] + h[1:]) / 2).astype(np.float32)  # exactly representable midpoints of neighbours
    vals = np.concatenate([vals, ties, -ties, np.float32([65504, 65520, 65519.99, 1e-8, 2.0**-25, 2.0**-24])])
    ours = np.array([L.orc_f2h(float(v)) for v in vals], dtype=np.uint16)
    with np.errstate(over="ignore"):
        ref = vals.astype(np.float16).view(np.uint16)
    assert np.array_equal(ours, ref)


# ---------------------------------------------------------------------------------------------
# Philox4x32-10 (Salmon et al., SC'11) -- Random123 known-answer vectors
# ---------------------------------------------------------------------------------------------
@pytest.mark.parametrize("ctr,key,expect", [
    ([0, 0, 0, 0], [0, 0], [0x6627E8D5, 0xE169C58D, 0xBC57AC4C, 0x9B00DBD8]),
    ([0xFFFFFFFF] * 4, [0xFFFFFFFF] * 2, [0x408F276D, 0x41C83B0E, 0xA20BC7C6, 0x6D5451FD]),
    ([0x243F6A88, 0x85A308D3, 0x13198A2E, 0x03707344], [0xA4093822, 0x299F31D0],
     [0xD16CFE09, 0x94FDCCEB, 0x5001E420, 0x24126EA1]),
])
def test_philox_kat(orc, ctr, key, expect):
    assert list(orc.philox(ctr, key)) == expect


def test_fnv1a_recurrence_and_reference_basis(orc):
    L = orc.lib()
    std_basis = 14695981039346656037
    # published FNV-1a 64-bit test vectors (Fowler/Noll/Vo)
    assert L.orc_fnv1a64_basis(b"", std_basis) == 0xCBF29CE484222325
    assert L.orc_fnv1a64_basis(b"a", std_basis) == 0xAF63DC4C8601EC8C
    assert L.orc_fnv1a64_basis(b"foobar", std_basis) == 0x85944171F73967E8
    # hash_string (Utils.cpp:9-16) starts from the reference's own basis 1469598103934665603
    assert L.orc_fnv1a64(b"") == 1469598103934665603
    assert L.orc_fnv1a64(b"a") == ((1469598103934665603 ^ 0x61) * 1099511628211) % 2**64


def test_random_ids_in_range(orc):
    ids = orc.random_ids(4096, 4096, 1)
    assert ids.min() >= 0 and ids.max() < 4096
    assert len(set(ids.tolist())) > 2500  # ~ 4096 * (1 - 1/e) distinct values expected


def test_fill_normal_moments(orc):
    x = orc.fill_normal(1 << 20, orc.F32, 0, "blk.0.attn_q.weight", 0.0, 0.02).astype(np.float64)
    assert abs(x.mean()) < 1e-4
    assert abs(x.std() - 0.02) < 1e-4
    # Box-Muller: the pair (z0, z1) of one uniform pair has norm sqrt(-2 ln u1) -- independent of u2
    kurt = ((x / x.std()) ** 4).mean()
    assert abs(kurt - 3.0) < 0.05


# ---------------------------------------------------------------------------------------------
# GGUF parsing (GGUFLoader.cpp:625-980) on files assembled byte by byte
# ---------------------------------------------------------------------------------------------
def _gstr(s):
    b = s.encode()
    return struct.pack("<Q", len(b)) + b


def build_gguf(tensors, kvs, convention="reference", align=32, pad_infos_to=None):
    """tensors: list of (name, dims, raw_type, data_bytes). Returns (bytes, data_start, offsets)."""
    out = bytearray()
    out += struct.pack("<IIQQ", 0x46554747, 3, len(tensors), len(kvs))
    for k, t, v in kvs:
        out += _gstr(k) + struct.pack("<I", t) + v
    offs, off = [], 0
    for name, dims, rt, data in tensors:
        offs.append(off)
        out += _gstr(name) + struct.pack("<I", len(dims)) + b"".join(struct.pack("<Q", d) for d in dims)
        out += struct.pack("<IQ", rt, off)
        off = (off + len(data) + align - 1) // align * align
    after = len(out)
    start = after if convention == "reference" else (after + align - 1) // align * align
    out += b"\0" * (start - after)
    for (name, dims, rt, data), o in zip(tensors, offs):
        out += b"\0" * (start + o - len(out))
        out += data
    return bytes(out), start, offs


def _open(orc, path):
    h = ctypes.c_void_p()
    rc = orc.lib().orc_gguf_open(str(path).encode(), ctypes.byref(h))
    return rc, h


def test_gguf_reference_layout(orc, tmp_path):
    L = orc.lib()
    a = np.arange(12, dtype=np.float32) * 0.5
    b = (np.arange(6, dtype=np.float32) - 2.5).astype(np.float16)
    kvs = [("llama.embedding_length", 4, struct.pack("<I", 64)),
           ("llama.rope.freq_base", 6, struct.pack("<f", 500000.0)),
           ("general.architecture", 8, _gstr("llama")),
           ("tokenizer.ggml.tokens", 9, struct.pack("<IQ", 8, 2) + _gstr("ab") + _gstr("c")),
           ("llama.block_count", 5, struct.pack("<i", 3))]  # INT32, not UINT32: reads as 0
    data, start, offs = build_gguf([("t.a", [4, 3], 6, a.tobytes()), ("t.b", [6], 48, b.tobytes())], kvs)
    p = tmp_path / "ref.gguf"
    p.write_bytes(data)
    rc, h = _open(orc, p)
    assert rc == 0
    try:
        assert L.orc_gguf_tensor_count(h) == 2 and L.orc_gguf_metadata_count(h) == 5
        assert L.orc_gguf_version(h) == 3
        assert L.orc_gguf_convention(h) == 0
        assert L.orc_gguf_data_start(h) == start  # no alignment padding (GGUFLoader.cpp:653)
        out = np.zeros(16, dtype=np.float32)
        assert L.orc_gguf_read_f32(h, b"t.a", orc.ptr(out), 16) == 12
        assert np.array_equal(out[:12], a)
        assert L.orc_gguf_read_f32(h, b"t.b", orc.ptr(out), 16) == 6
        assert np.array_equal(out[:6], b.astype(np.float32))
        idx = L.orc_gguf_find(h, b"t.b")
        nd, rt, do, ds = ctypes.c_uint32(), ctypes.c_uint32(), ctypes.c_uint64(), ctypes.c_uint64()
        dims = (ctypes.c_uint64 * 4)()
        L.orc_gguf_tensor_info(h, idx, None, 0, ctypes.byref(nd), dims, ctypes.byref(rt), ctypes.byref(do),
                               ctypes.byref(ds))
        assert (nd.value, rt.value, do.value, ds.value) == (1, 48, start + offs[1], 12)
        cfg = orc.Config()
        L.orc_gguf_model_config(h, ctypes.byref(cfg))
        assert cfg.hidden_size == 64 and cfg.rope_theta == 500000.0
        assert cfg.num_layers == 0  # get_uint32 on an INT32 value returns 0 (GGUFLoader.cpp:39-42)
        assert cfg.num_heads == 32 and cfg.num_kv_heads == 32  # defaults, kv defaults to heads
        assert L.orc_gguf_read_f32(h, b"missing", orc.ptr(out), 16) == -30
    finally:
        L.orc_gguf_close(h)


def test_gguf_ggml_layout_and_alignment(orc, tmp_path):
    L = orc.lib()
    a = np.linspace(-1, 1, 10, dtype=np.float32)
    b = np.linspace(-2, 2, 7, dtype=np.float32).astype(np.float16)
    kvs = [("general.alignment", 4, struct.pack("<I", 64))]
    data, start, offs = build_gguf([("x", [10], 0, a.tobytes()), ("y", [7], 1, b.tobytes())], kvs,
                                   convention="ggml", align=64)
    assert start % 64 == 0
    p = tmp_path / "ggml.gguf"
    p.write_bytes(data)
    rc, h = _open(orc, p)
    assert rc == 0
    try:
        assert L.orc_gguf_convention(h) == 1
        assert L.orc_gguf_data_start(h) == start
        out = np.zeros(16, dtype=np.float32)
        assert L.orc_gguf_read_f32(h, b"x", orc.ptr(out), 16) == 10 and np.array_equal(out[:10], a)
        assert L.orc_gguf_read_f32(h, b"y", orc.ptr(out), 16) == 7
        assert np.array_equal(out[:7], b.astype(np.float32))
    finally:
        L.orc_gguf_close(h)


def test_gguf_error_codes(orc, tmp_path):
    assert _open(orc, tmp_path / "nope.gguf")[0] == -1
    bad = tmp_path / "bad.gguf"
    bad.write_bytes(b"GGUX" + b"\0" * 40)
    assert _open(orc, bad)[0] == -2
    data, _, _ = build_gguf([("t", [4], 6, b"\0" * 16)], [("k", 8, _gstr("value"))])
    trunc_meta = tmp_path / "tm.gguf"
    trunc_meta.write_bytes(data[:24 + 8 + 1 + 4 + 3])  # cut inside the first metadata value
    assert _open(orc, trunc_meta)[0] == -3
    hdr = 24 + len(_gstr("k")) + 4 + len(_gstr("value"))
    trunc_info = tmp_path / "ti.gguf"
    trunc_info.write_bytes(data[:hdr + 10])  # cut inside the tensor info
    assert _open(orc, trunc_info)[0] == -4
    unknown = tmp_path / "unk.gguf"
    unknown.write_bytes(build_gguf([("t", [4], 6, b"\0" * 16)], [("k", 77, b"\0" * 4)])[0])
    assert _open(orc, unknown)[0] == -3  # read_value rejects unknown types (:976-978)


# ---------------------------------------------------------------------------------------------
# primitives: closed forms and invariants
# ---------------------------------------------------------------------------------------------
def test_rmsnorm_closed_form(orc):
    rng = np.random.default_rng(0)
    x = rng.normal(0, 3, 4096).astype(np.float32)
    y = orc.rmsnorm(x, np.ones(4096, np.float32), 0.0)
    assert abs(math.sqrt(float((y.astype(np.float64) ** 2).mean())) - 1.0) < 1e-6
    y2 = orc.rmsnorm(x * 7.5, np.ones(4096, np.float32), 0.0)
    assert np.allclose(y, y2, rtol=1e-6, atol=1e-6)
    g = rng.normal(0, 1, 4096).astype(np.float32)
    assert np.allclose(orc.rmsnorm(x, g, 0.0), y * g, rtol=1e-6, atol=1e-6)
    # eps enters under the square root: a constant vector c gives c / sqrt(c^2 + eps)
    c = np.full(8, 0.01, np.float32)
    assert np.allclose(orc.rmsnorm(c, None, 1e-4), 0.01 / math.sqrt(1e-4 + 1e-4), rtol=1e-6)


def test_rope_identity_norm_relative(orc):
    rng = np.random.default_rng(1)
    hd, nh, theta = 128, 3, 500000.0
    v = rng.normal(0, 1, nh * hd).astype(np.float32)
    assert np.array_equal(orc.rope(v, nh, hd, 0, theta), v)
    r = orc.rope(v, nh, hd, 777, theta)
    pairs = lambda a: (a.reshape(-1, 2).astype(np.float64) ** 2).sum(1)
    assert np.allclose(pairs(r), pairs(v), rtol=1e-5)
    q = rng.normal(0, 1, hd).astype(np.float32)
    k = rng.normal(0, 1, hd).astype(np.float32)
    d1 = float(np.dot(orc.rope(q, 1, hd, 50, theta).astype(np.float64), orc.rope(k, 1, hd, 20, theta)))
    d2 = float(np.dot(orc.rope(q, 1, hd, 1030, theta).astype(np.float64), orc.rope(k, 1, hd, 1000, theta)))
    assert abs(d1 - d2) < 1e-4 * max(1.0, abs(d1))


def test_rope_adjacent_pair_convention(orc):
    # head_dim 4, pos 3, base 10000: pair (0,1) rotates by 3 rad, pair (2,3) by 3 * 10000^(-2/4)
    v = np.array([1.0, 2.0, -0.5, 4.0], np.float32)
    out = orc.rope(v, 1, 4, 3, 10000.0)
    a0, a1 = 3.0, 3.0 * 10000.0 ** (-0.5)
    rot = lambda x, y, a: (x * math.cos(a) - y * math.sin(a), x * math.sin(a) + y * math.cos(a))
    exp = np.array([*rot(1.0, 2.0, a0), *rot(-0.5, 4.0, a1)], np.float32)
    assert np.allclose(out, exp, atol=1e-6)


def test_attention_closed_forms(orc):
    rng = np.random.default_rng(2)
    nq, nkv, hd, cap = 8, 2, 64, 16
    q = rng.normal(0, 1, nq * hd).astype(np.float32)
    kc = rng.normal(0, 1, (nkv, cap, hd)).astype(np.float32)
    vc = rng.normal(0, 1, (nkv, cap, hd)).astype(np.float32)
    # one key: output is that value, for every head of the group (kv_head = head * n_kv / n_q)
    out = orc.attention_decode(q, kc, vc, nq, nkv, hd, cap, 1, 0.125).reshape(nq, hd)
    for h in range(nq):
        assert np.allclose(out[h], vc[h * nkv // nq, 0], atol=1e-6)
    # identical keys: uniform weights -> mean of the values
    kc2 = np.repeat(kc[:, :1], cap, axis=1)
    out = orc.attention_decode(q, kc2, vc, nq, nkv, hd, cap, 11, 0.125).reshape(nq, hd)
    for h in range(nq):
        assert np.allclose(out[h], vc[h * nkv // nq, :11].mean(0), atol=1e-5)
    # a dominant key takes all the weight
    kc3 = kc.copy()
    kc3[:, 5] = q.reshape(nq, hd)[::nq // nkv] * 100
    out = orc.attention_decode(q, kc3, vc, nq, nkv, hd, cap, 9, 1.0).reshape(nq, hd)
    assert np.allclose(out[0], vc[0, 5], atol=1e-4)


@pytest.mark.parametrize("length,window,n_global,threshold,attended", [
    # threshold not passed (len <= threshold): every key 0..p
    (32, 8, 4, 32, list(range(32))),
    # p = 39: globals 0..3 and the window 31..39
    (40, 8, 4, 32, [0, 1, 2, 3] + list(range(31, 40))),
    # p = 13: window 5..13 and globals 0..3 leave out key 4 only
    (14, 8, 4, 8, [0, 1, 2, 3] + list(range(5, 14))),
    # window and globals overlap: 0..p
    (12, 8, 4, 8, list(range(12))),
    # no global tokens, window 0: the query attends to itself only
    (50, 0, 0, 1, [49]),
    # threshold 0: windowed from the first position on
    (64, 3, 2, 0, [0, 1, 60, 61, 62, 63]),
])
def test_windowed_attention_sets(orc, length, window, n_global, threshold, attended):
    """Equal keys give uniform weights, and the values are one-hot in the key position, so the
    output is exactly 1/|A| on the attended set A and 0 elsewhere."""
    nq, nkv, hd, cap = 4, 2, 64, 64
    rng = np.random.default_rng(7)
    q = rng.normal(0, 1, nq * hd).astype(np.float32)
    kc = np.repeat(rng.normal(0, 1, (nkv, 1, hd)).astype(np.float32), cap, axis=1)
    vc = np.zeros((nkv, cap, hd), np.float32)
    for t in range(cap):
        vc[:, t, t] = 1.0
    out = orc.attention_decode(q, kc, vc, nq, nkv, hd, cap, length, 0.125,
                               window=(window, n_global, threshold)).reshape(nq, hd)
    want = np.zeros(hd, np.float32)
    want[attended] = 1.0 / len(attended)
    for h in range(nq):
        assert np.allclose(out[h], want, atol=1e-7), (h, np.nonzero(out[h])[0])
    # keys outside the set (and their values) do not matter
    kc2, vc2 = kc.copy(), vc.copy()
    outside = [t for t in range(length) if t not in attended]
    kc2[:, outside] = rng.normal(0, 5, (nkv, len(outside), hd))
    vc2[:, outside] = rng.normal(0, 5, (nkv, len(outside), hd))
    out2 = orc.attention_decode(q, kc2, vc2, nq, nkv, hd, cap, length, 0.125,
                                window=(window, n_global, threshold)).reshape(nq, hd)
    assert np.array_equal(out, out2)
    # an unreached threshold is the dense kernel
    dense = orc.attention_decode(q, kc2, vc2, nq, nkv, hd, cap, length, 0.125)
    unreached = orc.attention_decode(q, kc2, vc2, nq, nkv, hd, cap, length, 0.125, window=(window, n_global, length))
    assert np.array_equal(dense, unreached)


def test_gemm_matches_numpy(orc):
    rng = np.random.default_rng(4)
    for (N, K, B) in [(64, 4096, 1), (96, 14336, 4), (40, 4096, 16)]:
        W = rng.normal(0, 0.02, (N, K)).astype(np.float16)
        X = rng.normal(0, 1, (K, B)).astype(np.float16).astype(np.float32)
        Y = orc.gemm_nt(W, X)
        ref = W.astype(np.float64) @ X.astype(np.float64)
        assert np.max(np.abs(Y - ref)) < 1e-5
    W32 = rng.normal(0, 0.02, (33, 688)).astype(np.float32)
    x = rng.normal(0, 1, 688).astype(np.float32)
    assert np.allclose(orc.gemm_nt(W32, x)[:, 0], W32.astype(np.float64) @ x, atol=1e-6)


def test_swiglu_closed_forms(orc):
    from scipy.special import expit
    g = np.array([0.0, 30.0, -30.0, 1.0, -2.0], np.float32)
    u = np.array([5.0, 2.0, 3.0, 1.0, 1.5], np.float32)
    h = orc.swiglu(g, u)
    assert h[0] == 0.0
    assert abs(h[1] - 60.0) < 1e-5 and abs(h[2]) < 1e-10
    assert np.allclose(h[3:], (g * expit(g) * u)[3:], rtol=1e-6)


# ---------------------------------------------------------------------------------------------
# samplers (VulkanSymbioteEngine.cpp:1540-1553, 1794-1855; Utils.cpp:140-184)
# ---------------------------------------------------------------------------------------------
def test_greedy_first_index_of_max(orc):
    lg = np.array([0.5, 2.0, -1.0, 2.0, 1.9], np.float32)
    assert orc.sample(lg, orc.SAMPLE_GREEDY) == 1
    assert orc.sample(np.full(7, -np.inf, np.float32), orc.SAMPLE_GREEDY) == 0
    assert orc.sample(np.array([np.nan, 5.0, 6.0], np.float32), orc.SAMPLE_GREEDY) == 0
    assert orc.sample(np.array([1.0, np.nan, 6.0], np.float32), orc.SAMPLE_GREEDY) == 2
    # T > 0 through the member top_k_sampling returns tokens[0]: the argmax of the probabilities
    rng = np.random.default_rng(5)
    for _ in range(20):
        l = rng.normal(0, 1.3, 4096).astype(np.float32)
        assert orc.sample(l, orc.SAMPLE_REFERENCE, 0.7) == int(np.argmax(l))
    # temperature <= 0 is greedy in every mode (sample_token :1541)
    l = rng.normal(0, 1, 100).astype(np.float32)
    assert orc.sample(l, orc.SAMPLE_TOPK_SEEDED, 0.0, 40, 9, 3) == int(np.argmax(l))


def test_topk_sampler_distribution(orc):
    """Empirical frequencies over many steps match softmax((l - max)/T) restricted to the top k."""
    rng = np.random.default_rng(6)
    l = rng.normal(0, 1.0, 500).astype(np.float32)
    T, k, n = 0.7, 5, 20000
    counts = np.zeros(500)
    for step in range(n):
        counts[orc.sample(l, orc.SAMPLE_TOPK_SEEDED, T, k, 1234, step)] += 1
    top = np.argsort(-l, kind="stable")[:k]
    p = np.exp((l[top] - l[top[0]]) / T)
    p /= p.sum()
    assert counts[np.setdiff1d(np.arange(500), top)].sum() == 0
    emp = counts[top] / n
    assert np.all(np.abs(emp - p) < 4 * np.sqrt(p * (1 - p) / n) + 1e-3)
    # k = 1 and vanishing temperature are the argmax
    assert all(orc.sample(l, orc.SAMPLE_TOPK_SEEDED, T, 1, 7, s) == int(np.argmax(l)) for s in range(20))
    assert all(orc.sample(l, orc.SAMPLE_TOPK_SEEDED, 1e-4, 40, 7, s) == int(np.argmax(l)) for s in range(20))
