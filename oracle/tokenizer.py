"""CPU restatement of Vulkan-Symbiote-Loader's tokenizer (text <-> ids).

TEST INFRASTRUCTURE ONLY (the oracle): loaded by tests/, never by the product.

Restates (paths relative to the reference repository root):
  - byte fallback vocabulary       vk_symbiote/src/Tokenizer.cpp:113-129 (256 one-byte tokens)
  - encode                         Tokenizer.cpp:131-178: words split on C-locale whitespace
                                   (std::istringstream >>); a word in the vocabulary is one id;
                                   otherwise one id per byte: the byte's one-byte token, or
                                   ((uint32)(signed char)b * 31) % 31000 + 1000; with no vocabulary
                                   at all, one hashed id per word; an empty result is [0]
  - decode                         Tokenizer.cpp:180-198: vocab[id % len(vocab)], joined by " "
  - vocabulary from GGUF metadata  the string array "tokenizer.ggml.tokens" (id = index), else the
                                   per-id string keys "tokenizer.ggml.tokens.<id>" that the
                                   reference's scan (Tokenizer.cpp:48-74) looks for: id = std::stoul
                                   of the text after the last '.', kept below 100000, the list
                                   resized to id + 1 at every key (it may shrink), the map entry
                                   value -> id written at every key; else the byte fallback.
                                   (The reference's own scan reads each key's value type before
                                   the key, :41-46, so it cannot read any real file; the layout it
                                   looks for is restated, not its misreads.)
Parity pins: tests/test_tokenizer.py (hand-computed ids, hash values, the resize rule, stoul
parsing, whitespace classes, files assembled byte by byte).
"""
import struct

WHITESPACE = b" \t\n\v\f\r"  # isspace() in the "C" locale
MAX_KEYED_ID = 100000


def split_words(text):
    """std::istringstream >> std::string: maximal runs of non-whitespace bytes."""
    words, cur = [], bytearray()
    for b in text:
        if b in WHITESPACE:
            if cur:
                words.append(bytes(cur))
                cur = bytearray()
        else:
            cur.append(b)
    if cur:
        words.append(bytes(cur))
    return words


def char_hash(b):
    """static_cast<uint32_t>(c) * 31 with c a signed char, then % 31000 + 1000 (Tokenizer.cpp:150-151)."""
    signed = b - 256 if b >= 128 else b
    return ((signed & 0xFFFFFFFF) * 31 & 0xFFFFFFFF) % 31000 + 1000


def word_hash(word):
    """Tokenizer.cpp:160-166: h = h * 31 + (unsigned char)c over the word, % 31000 + 1000."""
    h = 0
    for b in word:
        h = (h * 31 + b) & 0xFFFFFFFF
    return h % 31000 + 1000


def stoul_u32(s):
    """std::stoul(s) truncated to uint32_t; None where stoul throws (no digits, or out of range)."""
    i, n = 0, len(s)
    while i < n and s[i] in " \t\n\v\f\r":
        i += 1
    neg = False
    if i < n and s[i] in "+-":
        neg = s[i] == "-"
        i += 1
    j = i
    while j < n and s[j].isdigit() and s[j] in "0123456789":
        j += 1
    if j == i:
        return None
    v = int(s[i:j])
    if v > 0xFFFFFFFFFFFFFFFF:
        return None
    if neg:
        v = (-v) & 0xFFFFFFFFFFFFFFFF
    return v & 0xFFFFFFFF


class RefTokenizer:
    def __init__(self, vocab, token_map, source):
        self.vocab, self.map, self.source = vocab, token_map, source

    @classmethod
    def simple(cls):
        vocab = [bytes([i]) for i in range(256)]
        return cls(vocab, {t: i for i, t in enumerate(vocab)}, "bytes")

    @classmethod
    def from_tokens(cls, tokens):
        if not tokens:
            return cls.simple()
        m = {}
        for i, t in enumerate(tokens):
            m[t] = i  # a repeated string keeps its last id
        return cls(list(tokens), m, "array")

    @classmethod
    def from_keyed(cls, entries):
        """entries: (key suffix after the last '.', value bytes) in file order."""
        vocab, m = [], {}
        for suffix, value in entries:
            tid = stoul_u32(suffix)
            if tid is None or tid >= MAX_KEYED_ID:
                continue
            m[value] = tid
            vocab = (vocab + [b""] * (tid + 1 - len(vocab)))[:tid + 1]
            vocab[tid] = value
        if not m:
            return cls.simple()
        return cls(vocab, m, "keys")

    def encode(self, text):
        ids = []
        if self.map:
            for w in split_words(text):
                if w in self.map:
                    ids.append(self.map[w])
                    continue
                for b in w:
                    c = bytes([b])
                    ids.append(self.map[c] if c in self.map else char_hash(b))
        else:
            ids = [word_hash(w) for w in split_words(text)]
        return ids or [0]

    def decode(self, ids):
        if not self.vocab:
            return b""
        return b" ".join(self.vocab[i % len(self.vocab)] for i in ids)


# ---------------------------------------------------------------------------------------------
# GGUF metadata (header and key/value section only; GGUFLoader.cpp:625-663, :847-980)
# ---------------------------------------------------------------------------------------------
_SCALAR = {0: 1, 1: 1, 2: 2, 3: 2, 4: 4, 5: 4, 6: 4, 7: 1, 10: 8, 11: 8, 12: 8}


def _value(buf, o, t):
    if t in _SCALAR:
        return buf[o:o + _SCALAR[t]], o + _SCALAR[t]
    if t == 8:
        (n,) = struct.unpack_from("<Q", buf, o)
        return bytes(buf[o + 8:o + 8 + n]), o + 8 + n
    if t == 9:
        et, cnt = struct.unpack_from("<IQ", buf, o)
        o += 12
        items = []
        for _ in range(cnt):
            v, o = _value(buf, o, et)
            items.append(v)
        return (et, items), o
    raise ValueError(f"unknown metadata type {t}")


def metadata(path):
    """[(key, type, value)] in file order."""
    buf = open(path, "rb").read()
    magic, _ver, _nt, nkv = struct.unpack_from("<IIQQ", buf, 0)
    if magic != 0x46554747:
        raise ValueError("not a GGUF file")
    o, out = 24, []
    for _ in range(nkv):
        (kl,) = struct.unpack_from("<Q", buf, o)
        key = buf[o + 8:o + 8 + kl].decode("utf-8", "replace")
        (t,) = struct.unpack_from("<I", buf, o + 8 + kl)
        v, o = _value(buf, o + 12 + kl, t)
        out.append((key, t, v))
    return out


def from_gguf(path):
    try:
        kvs = metadata(path)
    except (OSError, ValueError, struct.error):
        return RefTokenizer.simple()
    for key, t, v in kvs:
        if key == "tokenizer.ggml.tokens" and t == 9 and v[0] == 8 and v[1]:
            return RefTokenizer.from_tokens(v[1])
    keyed = [(k[k.rfind(".") + 1:], v) for k, t, v in kvs
             if "tokenizer.ggml" in k and "tokens" in k and t == 8]
    return RefTokenizer.from_keyed(keyed)
