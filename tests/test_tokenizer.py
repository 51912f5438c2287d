"""Text path: the tokenizer behind encode / decode (vk_symbiote/src/Tokenizer.cpp:113-198).

The oracle restatement (oracle/tokenizer.py) is pinned by hand-computed ids: the byte fallback,
word / byte / hash lookups (hash values worked out by hand from (signed char * 31) % 31000 + 1000),
the keyed vocabulary's resize rule and std::stoul parsing, C-locale whitespace.  The product's
Tokenizer (C ABI) is then compared with the oracle on GGUF files assembled byte by byte, on files
from the product's writer, and on random byte strings.  CPU only.
"""
import struct

import numpy as np
import pytest

from oracle import tokenizer as otok
from test_oracle import build_gguf

VOCAB = [b"<unk>", b"<s>", b"</s>", b"hello", b"world", b"h", b"e", b"l", b"o", b"!"]


# ---------------------------------------------------------------------------------------------
# oracle pins
# ---------------------------------------------------------------------------------------------
def test_byte_fallback():
    t = otok.RefTokenizer.simple()
    assert t.encode(b"hello world") == list(b"helloworld")
    assert t.encode(b"") == [0] and t.encode(b" \t\n\v\f\r") == [0]
    assert t.encode("é".encode()) == [0xC3, 0xA9]             # bytes, not code points
    assert t.encode(b"a\vb\fc\rd") == [97, 98, 99, 100]         # every C-locale space splits
    assert t.decode([104, 105, 256 + 33]) == b"h i !"         # id % 256, joined by one space
    assert t.decode([]) == b""


def test_vocab_words_bytes_and_hash():
    t = otok.RefTokenizer.from_tokens(VOCAB)
    # "hello" is a word; "world!" is not: w -> hash 119*31 % 31000 + 1000 = 4689, o -> 8,
    # r -> 114*31 + 1000 = 4534, l -> 7, d -> 100*31 + 1000 = 4100, ! -> 9
    assert t.encode(b"hello world!") == [3, 4689, 8, 4534, 7, 4100, 9]
    assert t.encode(b"world") == [4]
    # bytes >= 0x80 widen with their sign: 0xC3 -> -61 -> 4294967235*31 mod 2^32 = 4294965405,
    # % 31000 = 8405 -> 9405; 0xA9 -> 8599; 0x80 -> 7328; 0xFF -> 11265
    assert t.encode("é".encode()) == [9405, 8599]
    assert t.encode(b"\x80\xff") == [7328, 11265]
    assert t.encode(b"   ") == [0]
    assert t.decode([3, 4, 13]) == b"hello world hello"      # 13 % 10 = 3
    rep = otok.RefTokenizer.from_tokens([b"a", b"b", b"a"])
    assert rep.encode(b"a") == [2]                            # the last id of a repeated string


def test_no_vocabulary_hashes_words():
    t = otok.RefTokenizer([], {}, "none")
    # (97*31 + 98) % 31000 + 1000 = 4105; (99*31 + 100) + 1000 = 4169
    assert t.encode(b"ab cd") == [4105, 4169]
    assert t.encode(b"") == [0]


def test_keyed_vocabulary_resize_rule():
    t = otok.RefTokenizer.from_keyed([("0", b"a"), ("5", b"b"), ("2", b"c")])
    # resize(1) [a]; resize(6) [a,,,,,b]; resize(3) [a,,c]: the later, smaller id shrinks the list
    assert t.vocab == [b"a", b"", b"c"]
    assert t.encode(b"b") == [5]                              # the map keeps b -> 5
    assert t.decode([5]) == b"c" and t.decode([1]) == b""
    assert otok.RefTokenizer.from_keyed([("x", b"a"), ("100000", b"b")]).source == "bytes"


@pytest.mark.parametrize("s,v", [(" 12", 12), ("7x", 7), ("x", None), ("+3", 3), ("-1", 0xFFFFFFFF),
                                 ("4294967296", 0), ("99999999999999999999", None), ("", None),
                                 ("00042", 42)])
def test_stoul(s, v):
    assert otok.stoul_u32(s) == v


# ---------------------------------------------------------------------------------------------
# files: oracle and product agree
# ---------------------------------------------------------------------------------------------
def _str_array(items):
    return struct.pack("<IQ", 8, len(items)) + b"".join(struct.pack("<Q", len(x)) + x for x in items)


def _kv_string(key, value):
    return (key, 8, struct.pack("<Q", len(value)) + value)


def _files(tmp_path):
    base = [("llama.embedding_length", 4, struct.pack("<I", 64))]
    t = [("t", [4], 6, b"\0" * 16)]
    spec = {
        "array": base + [("tokenizer.ggml.tokens", 9, _str_array(VOCAB))],
        "keys": base + [_kv_string("tokenizer.ggml.tokens.0", b"a"), _kv_string("tokenizer.ggml.tokens.5", b"hello"),
                        _kv_string("tokenizer.ggml.tokens.2", b"c"), _kv_string("tokenizer.ggml.tokens.x", b"zz"),
                        _kv_string("tokenizer.ggml.tokens.7q", b"!")],
        "both": base + [_kv_string("tokenizer.ggml.tokens.0", b"q"),
                        ("tokenizer.ggml.tokens", 9, _str_array([b"x", b"y", b"hello"]))],
        "none": base,
        "empty_array": base + [("tokenizer.ggml.tokens", 9, _str_array([]))],
        "int_array": base + [("tokenizer.ggml.tokens", 9, struct.pack("<IQ", 4, 2) + b"\1\0\0\0\2\0\0\0")],
    }
    out = {}
    for name, kvs in spec.items():
        p = tmp_path / f"{name}.gguf"
        p.write_bytes(build_gguf(t, kvs)[0])
        out[name] = p
    out["missing"] = tmp_path / "missing.gguf"
    return out


CORPUS = [b"", b"hello", b"hello world!", b"  hello\tworld\n", "héllo wörld".encode(), b"a c q x y hello",
          b"\x00\x01 \xff\xfe", b"!!!", b"c a"]


def _random_texts(seed, n=200):
    rng = np.random.default_rng(seed)
    alphabet = list(b"helowrd! acqxy\t\n") + [0xC3, 0xA9, 0x80, 0xFF, 0x00, 0x0B]
    return [bytes(rng.choice(alphabet, size=int(rng.integers(0, 24))).astype(np.uint8)) for _ in range(n)]


@pytest.mark.parametrize("name,source,size", [("array", "array", 10), ("keys", "keys", 8), ("both", "array", 3),
                                              ("none", "bytes", 256), ("empty_array", "bytes", 256),
                                              ("int_array", "bytes", 256), ("missing", "bytes", 256)])
def test_product_tokenizer_matches_oracle(vsl, tmp_path, name, source, size):
    p = _files(tmp_path)[name]
    ref = otok.from_gguf(p)
    assert ref.source == source and len(ref.vocab) == size
    with vsl.Tokenizer(p) as t:
        assert (t.source, t.vocab_size) == (source, size)
        for text in CORPUS + _random_texts(len(name)):
            assert t.encode(text).tolist() == ref.encode(text), text
        rng = np.random.default_rng(3)
        for _ in range(50):
            ids = rng.integers(0, 2 ** 32, size=int(rng.integers(0, 6)), dtype=np.uint64).astype(np.uint32)
            assert t.decode(ids) == ref.decode([int(i) for i in ids])


def test_keyed_file_values(vsl, tmp_path):
    p = _files(tmp_path)["keys"]
    with vsl.Tokenizer(p) as t:
        # ids 0 "a", 5 "hello", 2 "c" (shrinks to 3 entries), "x" skipped, "7q" -> 7 "!" (grows to 8)
        assert t.encode(b"hello a c !").tolist() == [5, 0, 2, 7]
        assert t.decode([5, 7, 1]) == b" ! "  # "" + " " + "!" + " " + "": vocab[5], vocab[1] emptied by the shrink


@pytest.mark.parametrize("keyed", [False, True])
def test_writer_vocabulary_roundtrip(vsl, tmp_path, keyed):
    cfg = dict(hidden_size=64, num_layers=1, num_heads=2, num_kv_heads=2, intermediate_size=128, vocab_size=300,
               max_position_embeddings=64, rope_theta=10000.0, rms_eps=1e-5, dtype=0)
    vocab = [b"<unk>", b"<s>", b"</s>"] + [bytes([i]) for i in range(32, 127)] + \
            [("w%d" % i).encode() for i in range(200)] + ["ünï".encode(), b"a b"]
    p = tmp_path / f"v{int(keyed)}.gguf"
    vsl.write_synthetic_gguf(p, cfg, seed=1, vocab=vocab, keyed=keyed)
    ref = otok.from_gguf(p)
    assert ref.vocab == vocab and ref.source == ("keys" if keyed else "array")
    with vsl.Tokenizer(p) as t:
        assert t.vocab_size == len(vocab)
        for text in CORPUS + [b"w1 w199 w200 ab", "ünï x".encode()] + _random_texts(7):
            assert t.encode(text).tolist() == ref.encode(text)
        assert t.decode([0, 3 + 65, len(vocab) + 3 + 72]) == ref.decode([0, 3 + 65, len(vocab) + 3 + 72])
