"""ctypes wrapper of the oracle (oracle/libvsl_oracle.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, the smoke() entry point and the cpu_baseline leg of
bench.py, as the oracle.  The product never imports it.
"""
import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libvsl_oracle.so")

F32, F16 = 0, 1
SAMPLE_GREEDY, SAMPLE_REFERENCE, SAMPLE_TOPK_SEEDED = 0, 1, 2


class Config(ctypes.Structure):
    _fields_ = [("hidden_size", ctypes.c_uint32), ("num_layers", ctypes.c_uint32), ("num_heads", ctypes.c_uint32),
                ("num_kv_heads", ctypes.c_uint32), ("intermediate_size", ctypes.c_uint32),
                ("vocab_size", ctypes.c_uint32), ("head_dim", ctypes.c_uint32),
                ("max_position_embeddings", ctypes.c_uint32), ("rope_theta", ctypes.c_float),
                ("rms_eps", ctypes.c_float)]


_P = ctypes.c_void_p
_U32, _U64, _I32, _F32 = ctypes.c_uint32, ctypes.c_uint64, ctypes.c_int, ctypes.c_float
_SIGS = {
    "orc_h2f": (_F32, [ctypes.c_uint16]),
    "orc_f2h": (ctypes.c_uint16, [_F32]),
    "orc_fnv1a64": (_U64, [ctypes.c_char_p]),
    "orc_fnv1a64_basis": (_U64, [ctypes.c_char_p, _U64]),
    "orc_philox4x32_10": (None, [_P, _P, _P]),
    "orc_num_threads": (_I32, []),
    "orc_set_num_threads": (None, [_I32]),
    "orc_gguf_open": (_I32, [ctypes.c_char_p, ctypes.POINTER(_P)]),
    "orc_gguf_close": (None, [_P]),
    "orc_gguf_tensor_count": (_U64, [_P]),
    "orc_gguf_metadata_count": (_U64, [_P]),
    "orc_gguf_version": (_U32, [_P]),
    "orc_gguf_data_start": (_U64, [_P]),
    "orc_gguf_convention": (_I32, [_P]),
    "orc_gguf_find": (_I32, [_P, ctypes.c_char_p]),
    "orc_gguf_tensor_info": (_I32, [_P, _I32, ctypes.c_char_p, ctypes.c_size_t, ctypes.POINTER(_U32),
                                    ctypes.POINTER(_U64), ctypes.POINTER(_U32), ctypes.POINTER(_U64),
                                    ctypes.POINTER(_U64)]),
    "orc_gguf_read_f32": (ctypes.c_int64, [_P, ctypes.c_char_p, _P, _U64]),
    "orc_dequant": (ctypes.c_int64, [_P, _U64, _U32, _I32, _U64, _P]),
    "orc_attention_decode_window": (None, [_P, _P, _P, _U32, _U32, _U32, _U32, _U32, _F32, _U32, _U32, _U32, _P]),
    "orc_model_set_window": (None, [_P, _U32, _U32, _U32]),
    "orc_gguf_get_u32": (_I32, [_P, ctypes.c_char_p, ctypes.POINTER(_U32)]),
    "orc_gguf_get_f32": (_I32, [_P, ctypes.c_char_p, ctypes.POINTER(_F32)]),
    "orc_gguf_model_config": (None, [_P, ctypes.POINTER(Config)]),
    "orc_model_new": (_P, [ctypes.POINTER(Config)]),
    "orc_model_free": (None, [_P]),
    "orc_model_set_tensor": (_I32, [_P, ctypes.c_char_p, _P, _I32, _I32]),
    "orc_model_from_gguf": (_I32, [ctypes.c_char_p, ctypes.POINTER(_P)]),
    "orc_model_config": (None, [_P, ctypes.POINTER(Config)]),
    "orc_model_check": (_I32, [_P]),
    "orc_state_new": (_P, [_P, _U32, _I32]),
    "orc_state_free": (None, [_P]),
    "orc_forward": (_I32, [_P, _P, _U32, _U32, _P]),
    "orc_state_reset": (None, [_P]),
    "orc_generate": (_I32, [_P, _P, _U32, _U32, _I32, _F32, _U32, _U64, _I32, _I32, _P, _P]),
    "orc_teacher_forced": (_I32, [_P, _P, _U32, _U32, _I32, _P]),
    "orc_rmsnorm": (None, [_P, _P, _U32, _F32, _P]),
    "orc_rope": (None, [_P, _U32, _U32, _U32, _F32]),
    "orc_gemm_nt": (None, [_P, _I32, _U32, _U32, _P, _U32, _P]),
    "orc_attention_decode": (None, [_P, _P, _P, _U32, _U32, _U32, _U32, _U32, _F32, _P]),
    "orc_swiglu": (None, [_P, _P, _U32, _P]),
    "orc_sample": (_U32, [_P, _U32, _I32, _F32, _U32, _U64, _U64]),
    "orc_fill_normal": (None, [_P, _I32, _U64, _U64, ctypes.c_char_p, _F32, _F32]),
    "orc_random_ids": (None, [_P, _U32, _U32, _U64, ctypes.c_char_p]),
}

_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            subprocess.run(["make", "-C", HERE], check=True, stdout=subprocess.DEVNULL)
        _lib = ctypes.CDLL(LIB_PATH)
        for n, (r, a) in _SIGS.items():
            f = getattr(_lib, n)
            f.restype = r
            f.argtypes = a
    return _lib


def ptr(a):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def set_threads(n):
    lib().orc_set_num_threads(int(n))


def num_threads():
    return lib().orc_num_threads()


def philox(ctr, key):
    c = np.ascontiguousarray(ctr, dtype=np.uint32)
    k = np.ascontiguousarray(key, dtype=np.uint32)
    o = np.zeros(4, dtype=np.uint32)
    lib().orc_philox4x32_10(ptr(c), ptr(k), ptr(o))
    return o


def random_ids(n, vocab, seed, name="prompt"):
    out = np.zeros(n, dtype=np.uint32)
    lib().orc_random_ids(ptr(out), n, vocab, seed, name.encode())
    return out


def fill_normal(n, dtype, seed, name, mean=0.0, std=0.02):
    out = np.empty(n, dtype=np.float16 if dtype == F16 else np.float32)
    lib().orc_fill_normal(ptr(out), dtype, n, seed, name.encode(), mean, std)
    return out


def config_dict(c):
    return {f: getattr(c, f) for f, _ in Config._fields_}


class Model:
    """A model held by the oracle: from a GGUF file or from host arrays by GGUF tensor name."""

    def __init__(self, gguf_path=None, config=None):
        self._keep = []
        L = lib()
        h = ctypes.c_void_p()
        if gguf_path is not None:
            rc = L.orc_model_from_gguf(str(gguf_path).encode(), ctypes.byref(h))
            if rc:
                raise RuntimeError(f"oracle cannot load {gguf_path}: {rc}")
        else:
            c = Config(**config)
            if not c.head_dim:
                c.head_dim = c.hidden_size // c.num_heads
            h = ctypes.c_void_p(L.orc_model_new(ctypes.byref(c)))
        self.h = h
        c = Config()
        L.orc_model_config(self.h, ctypes.byref(c))
        self.config = config_dict(c)

    def set_window(self, window, n_global, threshold):
        """Windowed attention from sequence length threshold + 1 on (threshold None: dense)."""
        lib().orc_model_set_window(self.h, window, n_global, 0xFFFFFFFF if threshold is None else threshold)

    def set_tensor(self, name, arr, copy=False):
        arr = np.ascontiguousarray(arr)
        dt = F16 if arr.dtype == np.float16 else F32
        if dt == F32 and arr.dtype != np.float32:
            arr = arr.astype(np.float32)
        if not copy:
            self._keep.append(arr)
        rc = lib().orc_model_set_tensor(self.h, name.encode(), ptr(arr), dt, int(copy))
        if rc:
            raise RuntimeError(f"oracle set_tensor({name}) -> {rc}")

    def check(self):
        return lib().orc_model_check(self.h)

    def generate(self, prompt, max_new, sampler=SAMPLE_GREEDY, temperature=0.0, top_k=40, seed=0,
                 stop_on_eos=False, kv_f16=False, logits=False):
        p = np.ascontiguousarray(prompt, dtype=np.uint32)
        toks = np.zeros(max(max_new, 1), dtype=np.uint32)
        lg = np.zeros((max(max_new, 1), self.config["vocab_size"]), dtype=np.float32) if logits else None
        n = lib().orc_generate(self.h, ptr(p), len(p), max_new, sampler, temperature, top_k, seed, int(stop_on_eos),
                               int(kv_f16), ptr(toks), ptr(lg))
        if n < 0:
            raise RuntimeError(f"orc_generate -> {n}")
        return (toks[:n], lg[:n]) if logits else toks[:n]

    def teacher_forced(self, ids, n_out, kv_f16=False):
        ids = np.ascontiguousarray(ids, dtype=np.uint32)
        out = np.zeros((n_out, self.config["vocab_size"]), dtype=np.float32)
        rc = lib().orc_teacher_forced(self.h, ptr(ids), len(ids), n_out, int(kv_f16), ptr(out))
        if rc:
            raise RuntimeError(f"orc_teacher_forced -> {rc}")
        return out

    def continuations(self, prompt, runs, kv_f16=False):
        """Several generations from one processed prompt (the prompt's positions are computed once).
        runs: list of dicts with n (tokens to generate) and optionally sampler, temperature, top_k, seed.
        Each run restarts at position len(prompt); positions past it are overwritten before they are
        read, so the runs are independent.  Returns [(tokens, logits)], logits [n][vocab]: the logits
        each token was sampled from (as generate(..., logits=True))."""
        L = lib()
        V = self.config["vocab_size"]
        n_max = max(r["n"] for r in runs)
        st = L.orc_state_new(self.h, len(prompt) + n_max, int(kv_f16))
        if not st:
            raise MemoryError("oracle state")
        try:
            first = np.zeros(V, np.float32)
            for i, t in enumerate(prompt):
                rc = L.orc_forward(self.h, st, int(t), i, ptr(first) if i == len(prompt) - 1 else None)
                if rc:
                    raise RuntimeError(f"orc_forward -> {rc}")
            out = []
            for r in runs:
                n = r["n"]
                toks = np.zeros(n, np.uint32)
                lg = np.zeros((n, V), np.float32)
                cur = first.copy()
                for t in range(n):
                    lg[t] = cur
                    toks[t] = sample(cur, r.get("sampler", SAMPLE_GREEDY), r.get("temperature", 0.0),
                                     r.get("top_k", 40), r.get("seed", 0), t)
                    if t + 1 < n and L.orc_forward(self.h, st, int(toks[t]), len(prompt) + t, ptr(cur)):
                        raise RuntimeError("orc_forward failed")
                out.append((toks, lg))
            return out
        finally:
            L.orc_state_free(st)

    def decode_rate(self, prompt, max_seconds=20.0, max_tokens=64, kv_f16=True):
        """Time the oracle's token loop on the host: the prompt is processed first (untimed), then
        greedy decode steps run until max_seconds or max_tokens.  Returns (tokens, seconds)."""
        import time
        L = lib()
        V = self.config["vocab_size"]
        st = L.orc_state_new(self.h, len(prompt) + max_tokens + 1, int(kv_f16))
        if not st:
            raise MemoryError("oracle state")
        lg = np.zeros(V, np.float32)
        try:
            for i, t in enumerate(prompt):
                rc = L.orc_forward(self.h, st, int(t), i, ptr(lg) if i == len(prompt) - 1 else None)
                if rc:
                    raise RuntimeError(f"orc_forward -> {rc}")
            pos, n, t0 = len(prompt), 0, time.perf_counter()
            while n < max_tokens and time.perf_counter() - t0 < max_seconds:
                tok = int(np.argmax(lg))
                if L.orc_forward(self.h, st, tok, pos, ptr(lg)):
                    raise RuntimeError("orc_forward failed")
                pos += 1
                n += 1
            return n, time.perf_counter() - t0
        finally:
            L.orc_state_free(st)

    def close(self):
        if self.h:
            lib().orc_model_free(self.h)
            self.h = None
            self._keep = []

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def rmsnorm(x, gamma, eps):
    x = np.ascontiguousarray(x, dtype=np.float32)
    g = None if gamma is None else np.ascontiguousarray(gamma, dtype=np.float32)
    y = np.empty_like(x)
    lib().orc_rmsnorm(ptr(x), ptr(g), x.size, eps, ptr(y))
    return y


def rope(v, n_heads, head_dim, pos, theta):
    v = np.array(v, dtype=np.float32, copy=True)
    lib().orc_rope(ptr(v), n_heads, head_dim, pos, theta)
    return v


def gemm_nt(W, X):
    """Y[N][B] = W[N][K] X[K][B] (W fp16 or fp32, X fp32)."""
    W = np.ascontiguousarray(W)
    dt = F16 if W.dtype == np.float16 else F32
    if dt == F32:
        W = W.astype(np.float32)
    X = np.ascontiguousarray(X, dtype=np.float32)
    if X.ndim == 1:
        X = X[:, None]
    N, K = W.shape
    B = X.shape[1]
    Y = np.empty((N, B), dtype=np.float32)
    lib().orc_gemm_nt(ptr(W), dt, N, K, ptr(X), B, ptr(Y))
    return Y


def attention_decode(q, kc, vc, n_q, n_kv, hd, cap, length, scale, window=None):
    """window: None (dense) or (window, n_global, threshold)."""
    q = np.ascontiguousarray(q, dtype=np.float32)
    kc = np.ascontiguousarray(kc, dtype=np.float32)
    vc = np.ascontiguousarray(vc, dtype=np.float32)
    out = np.empty(n_q * hd, dtype=np.float32)
    if window is None:
        lib().orc_attention_decode(ptr(q), ptr(kc), ptr(vc), n_q, n_kv, hd, cap, length, scale, ptr(out))
    else:
        w, g, t = window
        lib().orc_attention_decode_window(ptr(q), ptr(kc), ptr(vc), n_q, n_kv, hd, cap, length, scale, w, g, t,
                                          ptr(out))
    return out


def swiglu(g, u):
    g = np.ascontiguousarray(g, dtype=np.float32)
    u = np.ascontiguousarray(u, dtype=np.float32)
    h = np.empty_like(g)
    lib().orc_swiglu(ptr(g), ptr(u), g.size, ptr(h))
    return h


def sample(logits, sampler, temperature=0.0, top_k=40, seed=0, step=0):
    lg = np.ascontiguousarray(logits, dtype=np.float32)
    return lib().orc_sample(ptr(lg), lg.size, sampler, temperature, top_k, seed, step)
