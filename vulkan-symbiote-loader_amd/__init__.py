"""Python binding of the MI355X backend for Vulkan-Symbiote-Loader's token loop.

A thin ctypes layer over the two C ABIs (include/vsl_hip.h, include/vsl_engine.h):
  * Engine           -- VulkanSymbioteEngine (vk_symbiote/include/vk_symbiote/VulkanSymbioteEngine.h:72-118):
                        open a GGUF or a synthetic model, generate from token ids or text, config,
                        benchmark, HBM/KV statistics, device->host copies of resident packs.
  * write_synthetic_gguf -- the seeded Llama-style GGUF writer.
  * hip()            -- the raw kernel-layer library with argtypes set (ops, arena, graphs).

The native libraries are built in-tree (build.py) and loaded from ./lib.  There is no fallback:
if they are missing, every entry point raises.
"""
import ctypes
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_DIR = os.path.join(_HERE, "lib")
HIP_LIB = os.path.join(LIB_DIR, "libvsl_hip.so")
ENGINE_LIB = os.path.join(LIB_DIR, "libvsl_engine.so")

VSL_OK, VSL_E_INVALID, VSL_E_HIP, VSL_E_OOM, VSL_E_UNSUPPORTED, VSL_E_CAPACITY = 0, -100, -101, -102, -103, -104
VSL_DT_F32, VSL_DT_F16, VSL_DT_F16X2, VSL_DT_F16F8 = 0, 1, 2, 3
VSL_DT_Q8_0, VSL_DT_Q4_0, VSL_DT_Q4_1 = 4, 5, 6  # resident block-quantized weight packs
VSL_WF_F32, VSL_WF_F16, VSL_WF_Q4_0, VSL_WF_Q4_1, VSL_WF_Q8_0 = 0, 1, 2, 3, 4
VSL_QL_REFERENCE, VSL_QL_GGML = 0, 1
GEMM_A_X2, GEMM_C_X2, GEMM_A_F8, GEMM_C_F8 = 0x100, 0x200, 0x400, 0x800


def GEMM_B8_SHIFT(s):
    """VSL_GEMM_B8_SHIFT(s): the weight shift of the fp8 lo product (B rounded to e4m3 as B * 2^s)."""
    return ((s + 128) & 0xFF) << 16
SAMPLE_GREEDY, SAMPLE_REFERENCE, SAMPLE_TOPK_SEEDED = 0, 1, 2
MAX_TOP_K = 262144  # VSL_MAX_TOP_K: the seeded top-k serves 1 <= min(top_k, V) <= MAX_TOP_K
EPI_STORE_F32, EPI_STORE_F16, EPI_RESID, EPI_SWIGLU = 0, 1, 2, 3
_MODES = {"greedy": SAMPLE_GREEDY, "reference": SAMPLE_REFERENCE, "topk": SAMPLE_TOPK_SEEDED}


class VslError(RuntimeError):
    def __init__(self, code, msg):
        super().__init__(f"{msg} (code {code})")
        self.code = code


class ModelSpec(ctypes.Structure):
    _fields_ = [("hidden_size", ctypes.c_uint32), ("num_layers", ctypes.c_uint32), ("num_heads", ctypes.c_uint32),
                ("num_kv_heads", ctypes.c_uint32), ("intermediate_size", ctypes.c_uint32),
                ("vocab_size", ctypes.c_uint32), ("max_position_embeddings", ctypes.c_uint32),
                ("rope_theta", ctypes.c_float), ("rms_eps", ctypes.c_float), ("init_std", ctypes.c_float),
                ("dtype", ctypes.c_uint32), ("head_dim", ctypes.c_uint32)]


class PackInfo(ctypes.Structure):
    _fields_ = [("pack_id", ctypes.c_uint64), ("type", ctypes.c_int32), ("layer_idx", ctypes.c_uint32),
                ("head_idx", ctypes.c_uint32), ("alignment", ctypes.c_uint32), ("compressed_size", ctypes.c_uint64),
                ("decompressed_size", ctypes.c_uint64), ("file_offset", ctypes.c_uint64),
                ("base_priority", ctypes.c_float), ("tier", ctypes.c_int32), ("dtype", ctypes.c_int32),
                ("n_dimensions", ctypes.c_uint32), ("resident_bytes", ctypes.c_uint64),
                ("device_ptr", ctypes.c_void_p)]


class EngineOptions(ctypes.Structure):
    _fields_ = [("device", ctypes.c_int32), ("kv_capacity", ctypes.c_uint32), ("use_graph", ctypes.c_uint32),
                ("prefill_chunk", ctypes.c_uint32), ("attn_splits", ctypes.c_uint32),
                ("batched_prefill", ctypes.c_uint32), ("prefill_split", ctypes.c_uint32),
                ("dequant_f32", ctypes.c_uint32), ("sparse_attention", ctypes.c_uint32),
                ("sparse_window", ctypes.c_uint32), ("sparse_global", ctypes.c_uint32),
                ("sparse_threshold", ctypes.c_uint32), ("prefill_lo8", ctypes.c_uint32),
                ("quant_decode", ctypes.c_uint32)]


class GenParams(ctypes.Structure):
    _fields_ = [("mode", ctypes.c_int32), ("temperature", ctypes.c_float), ("top_k", ctypes.c_uint32),
                ("stop_on_eos", ctypes.c_uint32), ("seed", ctypes.c_uint64)]


class GenStats(ctypes.Structure):
    _fields_ = [("prompt_tokens", ctypes.c_uint32), ("generated_tokens", ctypes.c_uint32),
                ("kv_positions", ctypes.c_uint32), ("pad", ctypes.c_uint32), ("prefill_ms", ctypes.c_double),
                ("decode_ms", ctypes.c_double)]


class PoolStats(ctypes.Structure):
    _fields_ = [("total_size", ctypes.c_uint64), ("used_size", ctypes.c_uint64), ("free_size", ctypes.c_uint64),
                ("allocation_count", ctypes.c_uint32), ("fragmentation_ratio", ctypes.c_float)]


class Sampler(ctypes.Structure):
    _fields_ = [("mode", ctypes.c_int32), ("temperature", ctypes.c_float), ("top_k", ctypes.c_uint32),
                ("pad", ctypes.c_uint32), ("seed", ctypes.c_uint64)]


class Ctrl(ctypes.Structure):
    _fields_ = [(n, ctypes.c_uint32) for n in
                ("pos", "step", "done", "stop_on_eos", "max_steps", "token", "capacity", "error")]


# model configurations named by the workloads they run
TINY = dict(hidden_size=256, num_layers=2, num_heads=4, num_kv_heads=4, intermediate_size=688, vocab_size=4096,
            max_position_embeddings=2048, rope_theta=10000.0, rms_eps=1e-5, dtype=VSL_DT_F32)
LLAMA_1B = dict(hidden_size=2048, num_layers=16, num_heads=32, num_kv_heads=8, intermediate_size=8192,
                vocab_size=32000, max_position_embeddings=4096, rope_theta=10000.0, rms_eps=1e-5, dtype=VSL_DT_F16)
LLAMA_8B = dict(hidden_size=4096, num_layers=32, num_heads=32, num_kv_heads=8, intermediate_size=14336,
                vocab_size=32000, max_position_embeddings=32768, rope_theta=500000.0, rms_eps=1e-5, dtype=VSL_DT_F16)

_P = ctypes.c_void_p
_U32, _U64, _I32, _F32 = ctypes.c_uint32, ctypes.c_uint64, ctypes.c_int, ctypes.c_float
_HIP_SIGS = {
    "vsl_last_error": (ctypes.c_char_p, []),
    "vsl_device_count": (_I32, [ctypes.POINTER(ctypes.c_int)]),
    "vsl_set_device": (_I32, [_I32]),
    "vsl_device_sync": (_I32, []),
    "vsl_arena_create": (_I32, [_I32, _U64, ctypes.POINTER(_P)]),
    "vsl_weight_bytes": (_U64, [_I32, _U64]),
    "vsl_gemm_f16_ws": (_I32, [_P, _P, _U32, _U32, _U32, _P, _I32, _P, _U64, _P]),
    "vsl_gemm_f16_ws_bytes": (_U64, [_U32, _U32, _U32, _I32]),
    "vsl_gemm_f16_direct": (_I32, [_U32, _U32, _U32, _I32]),
    "vsl_gemm_b8_shift": (_I32, [_F32]),
    "vsl_absmax_f16": (_I32, [_P, _U64, _P, _P]),
    "vsl_convert_weights": (_I32, [_P, _I32, _I32, _U64, _P, _I32, _P]),
    "vsl_attn_decode_window": (_I32, [_P, _P, _P, _I32, _U32, _U32, _U32, _U32, _F32, _U32, _P, _P, _P, _P,
                                      _U32, _U32, _U32, _P]),
    "vsl_attn_prefill_window": (_I32, [_P, _I32, _P, _P, _U32, _U32, _U32, _U32, _U32, _U32, _F32, _P, _I32,
                                       _U32, _U32, _U32, _P]),
    "vsl_arena_destroy": (_I32, [_P]),
    "vsl_arena_alloc": (_I32, [_P, _U64, _U64, ctypes.POINTER(_P)]),
    "vsl_arena_free": (_I32, [_P, _P]),
    "vsl_arena_reset": (_I32, [_P]),
    "vsl_arena_stats": (_I32, [_P, ctypes.POINTER(PoolStats)]),
    "vsl_arena_base": (_P, [_P]),
    "vsl_host_pinned_alloc": (_I32, [_U64, ctypes.POINTER(_P)]),
    "vsl_host_pinned_free": (_I32, [_P]),
    "vsl_stream_create": (_I32, [ctypes.POINTER(_P)]),
    "vsl_stream_destroy": (_I32, [_P]),
    "vsl_stream_sync": (_I32, [_P]),
    "vsl_event_create": (_I32, [ctypes.POINTER(_P)]),
    "vsl_event_destroy": (_I32, [_P]),
    "vsl_event_record": (_I32, [_P, _P]),
    "vsl_event_sync": (_I32, [_P]),
    "vsl_stream_wait_event": (_I32, [_P, _P]),
    "vsl_event_elapsed_ms": (_I32, [_P, _P, ctypes.POINTER(ctypes.c_float)]),
    "vsl_pack_upload": (_I32, [_P, _P, _U64, _P, _P]),
    "vsl_copy_d2h": (_I32, [_P, _P, _U64, _P]),
    "vsl_copy_h2d": (_I32, [_P, _P, _U64, _P]),
    "vsl_copy_d2d": (_I32, [_P, _P, _U64, _P]),
    "vsl_memset_d": (_I32, [_P, _I32, _U64, _P]),
    "vsl_fill_normal": (_I32, [_P, _I32, _U64, _U64, ctypes.c_char_p, _F32, _F32, _P]),
    "vsl_fill_const": (_I32, [_P, _I32, _U64, _F32, _P]),
    "vsl_embed": (_I32, [_P, _I32, _U32, _U32, _P, _U32, _P, _P]),
    "vsl_rmsnorm": (_I32, [_P, _P, _U32, _U32, _F32, _P, _I32, _P]),
    "vsl_gemv": (_I32, [_P, _I32, _U32, _U32, _P, _I32, _U32, _P, _I32, _P]),
    "vsl_gemv_batched": (_I32, [_P, _U32, _U32, _P, _U32, _P, _I32, _P]),
    "vsl_qkv_rope_append": (_I32, [_P, _P, _F32, _P, _I32, _U32, _U32, _U32, _U32, _P, _P, _P, _P, _I32, _U32, _P,
                                   _P, _P]),
    "vsl_attn_decode": (_I32, [_P, _P, _P, _I32, _U32, _U32, _U32, _U32, _F32, _U32, _P, _P, _P, _P, _P]),
    "vsl_attn_decode_noalloc": (_I32, [_P, _P, _P, _I32, _U32, _U32, _U32, _U32, _F32, _U32, _P, _P, _P]),
    "vsl_gemv_residual": (_I32, [_P, _I32, _U32, _U32, _P, _P, _P, _P]),
    "vsl_quant_pack_bytes": (ctypes.c_uint64, [_I32, _U32, _U32]),
    "vsl_quant_pack": (_I32, [_P, _I32, _I32, ctypes.c_uint64, _P, _U32, _U32, ctypes.c_uint64, _P]),
    "vsl_quantize_pack": (_I32, [_P, _I32, _U32, _U32, _I32, _P, _P]),
    "vsl_dequant_pack": (_I32, [_P, _I32, _U32, _U32, _P, _I32, _P]),
    "vsl_norm_swiglu": (_I32, [_P, _P, _F32, _P, _I32, _U32, _U32, _P, _P, _P]),
    "vsl_lm_head_sample": (_I32, [_P, _F32, _P, _I32, _U32, _U32, _P, _P, _I32, _P, Sampler, _P, _P, _P, _P, _P]),
    "vsl_lm_head_ws_blocks": (_U32, []),
    "vsl_sample_logits": (_I32, [_P, _U32, Sampler, _U64, _P, _P]),
    "vsl_ctrl_reset": (_I32, [_P, _U32, _U32, _U32, _U32, _P]),
    "vsl_gemm_f16": (_I32, [_P, _P, _U32, _U32, _U32, _P, _I32, _P]),
    "vsl_rope_split_append": (_I32, [_P, _U32, _U32, _U32, _U32, _U32, _P, _P, _P, _I32, _P, _P, _I32, _U32, _P]),
    "vsl_gemm_f16_qkv_rope_append": (_I32, [_P, _P, _U32, _U32, _I32, _U32, _U32, _U32, _U32, _P, _P, _P, _I32, _P,
                                             _P, _I32, _U32, _P, _P, _U64, _P]),
    "vsl_gemm_f16_resid_rmsnorm": (_I32, [_P, _P, _U32, _U32, _U32, _I32, _P, _P, _F32, _P, _I32, _P, _U64, _P]),
    "vsl_attn_prefill": (_I32, [_P, _I32, _P, _P, _U32, _U32, _U32, _U32, _U32, _U32, _F32, _P, _I32, _P]),
    "vsl_graph_begin": (_I32, [_P]),
    "vsl_graph_end": (_I32, [_P, ctypes.POINTER(_P)]),
    "vsl_graph_launch": (_I32, [_P, _P]),
    "vsl_graph_destroy": (_I32, [_P]),
}
_ENGINE_SIGS = {
    "vsl_engine_default_options": (None, [ctypes.POINTER(EngineOptions)]),
    "vsl_engine_last_error": (ctypes.c_char_p, []),
    "vsl_engine_open": (_I32, [ctypes.c_char_p, ctypes.POINTER(EngineOptions), ctypes.POINTER(_P)]),
    "vsl_engine_open_synthetic": (_I32, [ctypes.POINTER(ModelSpec), _U64, ctypes.POINTER(EngineOptions),
                                         ctypes.POINTER(_P)]),
    "vsl_engine_close": (_I32, [_P]),
    "vsl_engine_generate_ids": (_I32, [_P, _P, _U32, _U32, ctypes.POINTER(GenParams), _P, _P,
                                       ctypes.POINTER(_U32)]),
    "vsl_engine_generate_forced": (_I32, [_P, _P, _U32, _P, _U32, _U32, ctypes.POINTER(GenParams), _P, _P,
                                          ctypes.POINTER(_U32)]),
    "vsl_engine_generate_text": (_I32, [_P, ctypes.c_char_p, _U32, _F32, ctypes.c_char_p, _U64,
                                        ctypes.POINTER(_U64)]),
    "vsl_engine_begin": (_I32, [_P, _P, _U32, _U32, ctypes.POINTER(GenParams)]),
    "vsl_engine_decode": (_I32, [_P, _U32, ctypes.POINTER(_U32)]),
    "vsl_engine_sync": (_I32, [_P]),
    "vsl_engine_finish": (_I32, [_P, _P, ctypes.POINTER(_U32)]),
    "vsl_engine_time_op": (_I32, [_P, _I32, _U32, ctypes.POINTER(ctypes.c_double)]),
    "vsl_engine_get_config": (_I32, [_P, ctypes.POINTER(ModelSpec)]),
    "vsl_engine_last_stats": (_I32, [_P, ctypes.POINTER(GenStats)]),
    "vsl_engine_vram_stats": (_I32, [_P, ctypes.POINTER(PoolStats)]),
    "vsl_engine_kv_bytes": (_I32, [_P, ctypes.POINTER(_U64)]),
    "vsl_engine_weight_bytes": (_I32, [_P, ctypes.POINTER(_U64)]),
    "vsl_engine_clear_kv": (_I32, [_P]),
    "vsl_engine_benchmark": (_I32, [_P, _U32, _U32, _U32, ctypes.POINTER(ctypes.c_double),
                                    ctypes.POINTER(ctypes.c_double), ctypes.POINTER(ctypes.c_double)]),
    "vsl_engine_read_tensor": (_I32, [_P, ctypes.c_char_p, _P, _U64, ctypes.POINTER(ctypes.c_int)]),
    "vsl_write_synthetic_gguf": (_I32, [ctypes.c_char_p, ctypes.POINTER(ModelSpec), _U64, _I32]),
    "vsl_write_synthetic_gguf_vocab": (_I32, [ctypes.c_char_p, ctypes.POINTER(ModelSpec), _U64, _I32,
                                              ctypes.POINTER(ctypes.c_char_p), ctypes.POINTER(_U64), _U32, _I32]),
    "vsl_engine_pack_count": (_I32, [_P, ctypes.POINTER(_U64)]),
    "vsl_engine_pack": (_I32, [_P, _U64, ctypes.POINTER(PackInfo), ctypes.c_char_p, _U64]),
    "vsl_gguf_pack_count": (_I32, [_P, ctypes.POINTER(_U64)]),
    "vsl_gguf_pack": (_I32, [_P, _U64, ctypes.POINTER(PackInfo), ctypes.c_char_p, _U64]),
    "vsl_tokenizer_open": (_I32, [ctypes.c_char_p, ctypes.POINTER(_P)]),
    "vsl_tokenizer_close": (_I32, [_P]),
    "vsl_tokenizer_info": (_I32, [_P, ctypes.POINTER(_U32), ctypes.POINTER(ctypes.c_int)]),
    "vsl_tokenizer_encode": (_I32, [_P, ctypes.c_char_p, _U64, _P, _U64, ctypes.POINTER(_U64)]),
    "vsl_tokenizer_decode": (_I32, [_P, _P, _U64, _P, _U64, ctypes.POINTER(_U64)]),
    "vsl_synthetic_fill_host": (_I32, [_P, _I32, _U64, _U64, ctypes.c_char_p, _F32, _F32]),
    "vsl_gguf_open": (_I32, [ctypes.c_char_p, ctypes.POINTER(_P)]),
    "vsl_gguf_close": (_I32, [_P]),
    "vsl_gguf_info": (_I32, [_P, ctypes.POINTER(_U64), ctypes.POINTER(_U64), ctypes.POINTER(_U32),
                             ctypes.POINTER(ctypes.c_int), ctypes.POINTER(_U64)]),
    "vsl_gguf_model_config": (_I32, [_P, ctypes.POINTER(ModelSpec)]),
    "vsl_gguf_tensor": (_I32, [_P, ctypes.c_char_p, ctypes.POINTER(_U64), ctypes.POINTER(_U64), ctypes.POINTER(_U32),
                               ctypes.POINTER(_U32), ctypes.POINTER(_U64)]),
    "vsl_gguf_read_f32": (ctypes.c_int64, [_P, ctypes.c_char_p, _P, _U64]),
    "vsl_config_load_args": (_I32, [_I32, ctypes.POINTER(ctypes.c_char_p)]),
    "vsl_config_load_file": (_I32, [ctypes.c_char_p]),
    "vsl_config_save_file": (_I32, [ctypes.c_char_p]),
    "vsl_config_reset": (_I32, []),
    "vsl_config_get": (_I32, [ctypes.POINTER(ctypes.c_int), ctypes.POINTER(ctypes.c_int), ctypes.POINTER(_U32),
                              ctypes.POINTER(_U64), ctypes.POINTER(ctypes.c_float)]),
}

_libs = {}


def _load(path, sigs):
    if not os.path.exists(path):
        raise OSError(f"native library {path} is not built; run vulkan-symbiote-loader_amd/build.py "
                      "(this backend has no non-native fallback)")
    lib = ctypes.CDLL(path, mode=ctypes.RTLD_GLOBAL)
    for name, (res, args) in sigs.items():
        f = getattr(lib, name)
        f.restype = res
        f.argtypes = args
    return lib


def hip():
    """The kernel-layer library (include/vsl_hip.h) with argtypes configured."""
    if "hip" not in _libs:
        _libs["hip"] = _load(HIP_LIB, _HIP_SIGS)
    return _libs["hip"]


def engine_lib():
    """The engine library (include/vsl_engine.h) with argtypes configured."""
    if "engine" not in _libs:
        hip()
        _libs["engine"] = _load(ENGINE_LIB, _ENGINE_SIGS)
    return _libs["engine"]


def check(rc, lib=None):
    if rc != 0:
        lib = lib or hip()
        msg = (lib.vsl_engine_last_error() if hasattr(lib, "vsl_engine_last_error") else lib.vsl_last_error())
        raise VslError(rc, (msg or b"").decode(errors="replace"))


def _ptr(a):
    return a.ctypes.data_as(ctypes.c_void_p)


def make_spec(cfg, init_std=0.02):
    s = ModelSpec()
    for k, v in cfg.items():
        setattr(s, k, v)
    s.init_std = init_std
    return s


def write_synthetic_gguf(path, cfg, seed=0, convention="reference", init_std=0.02, vocab=None, keyed=False):
    """cfg["dtype"]: VSL_WF_* storage of the 2-D weights. vocab: optional list of token strings or
    bytes, written as the array tokenizer.ggml.tokens (keyed=True: one key tokenizer.ggml.tokens.<id>
    per token)."""
    lib = engine_lib()
    spec = make_spec(cfg, init_std)
    conv = {"reference": 0, "ggml": 1}[convention]
    if vocab is None:
        check(lib.vsl_write_synthetic_gguf(str(path).encode(), ctypes.byref(spec), seed, conv), lib)
        return
    toks = [t if isinstance(t, bytes) else t.encode() for t in vocab]
    arr = (ctypes.c_char_p * max(len(toks), 1))(*toks)
    lens = (_U64 * max(len(toks), 1))(*[len(t) for t in toks])
    check(lib.vsl_write_synthetic_gguf_vocab(str(path).encode(), ctypes.byref(spec), seed, conv, arr, lens,
                                             len(toks), int(bool(keyed))), lib)


class Tokenizer:
    """Tokenizer::from_gguf (path) or the 256-byte fallback (path None). Text is bytes or str (UTF-8)."""

    SOURCES = ("bytes", "array", "keys")

    def __init__(self, gguf_path=None):
        self._lib = engine_lib()
        h = ctypes.c_void_p()
        check(self._lib.vsl_tokenizer_open(None if gguf_path is None else str(gguf_path).encode(), ctypes.byref(h)),
              self._lib)
        self._h = h
        v, src = _U32(), ctypes.c_int()
        check(self._lib.vsl_tokenizer_info(self._h, ctypes.byref(v), ctypes.byref(src)), self._lib)
        self.vocab_size, self.source = v.value, self.SOURCES[src.value]

    def encode(self, text):
        b = text if isinstance(text, bytes) else text.encode()
        n = _U64()
        check(self._lib.vsl_tokenizer_encode(self._h, b, len(b), None, 0, ctypes.byref(n)), self._lib)
        out = np.zeros(max(n.value, 1), dtype=np.uint32)
        check(self._lib.vsl_tokenizer_encode(self._h, b, len(b), _ptr(out), n.value, ctypes.byref(n)), self._lib)
        return out[:n.value]

    def decode(self, ids):
        ids = np.ascontiguousarray(ids, dtype=np.uint32)
        n = _U64()
        check(self._lib.vsl_tokenizer_decode(self._h, _ptr(ids), ids.size, None, 0, ctypes.byref(n)), self._lib)
        buf = ctypes.create_string_buffer(max(n.value, 1))
        check(self._lib.vsl_tokenizer_decode(self._h, _ptr(ids), ids.size, buf, n.value, ctypes.byref(n)), self._lib)
        return buf.raw[:n.value]

    def close(self):
        if self._h:
            self._lib.vsl_tokenizer_close(self._h)
            self._h = None

    def __enter__(self):
        return self

    def __exit__(self, *a):
        self.close()


def synthetic_fill_host(n, dtype, seed, name, mean=0.0, std=0.02):
    out = np.empty(n, dtype=np.float16 if dtype == VSL_DT_F16 else np.float32)
    lib = engine_lib()
    check(lib.vsl_synthetic_fill_host(_ptr(out), dtype, n, seed, name.encode(), mean, std), lib)
    return out


class Engine:
    """VulkanSymbioteEngine on one MI355X."""

    def __init__(self, gguf_path=None, spec=None, seed=0, device=0, kv_capacity=0, use_graph=True,
                 prefill_chunk=0, attn_splits=0, batched_prefill=True, init_std=0.02, prefill_split=None,
                 dequant_f32=False, window=None, prefill_lo8=None, quant_decode=True):
        """window: None (dense attention) or (sparse_window, sparse_global, sparse_threshold) for the
        windowed long-context mode; (512, 16, 8192) are the reference's values. prefill_split /
        prefill_lo8: None keeps vsl_engine_default_options' stage masks."""
        self._lib = engine_lib()
        opt = EngineOptions()
        self._lib.vsl_engine_default_options(ctypes.byref(opt))
        opt.device, opt.kv_capacity, opt.use_graph = device, kv_capacity, int(bool(use_graph))
        opt.prefill_chunk, opt.attn_splits, opt.batched_prefill = prefill_chunk, attn_splits, int(bool(batched_prefill))
        if prefill_split is not None:
            opt.prefill_split = prefill_split
        if prefill_lo8 is not None:
            opt.prefill_lo8 = prefill_lo8
        opt.dequant_f32 = int(bool(dequant_f32))
        opt.quant_decode = int(bool(quant_decode))
        if window is not None:
            opt.sparse_attention = 1
            opt.sparse_window, opt.sparse_global, opt.sparse_threshold = window
        h = ctypes.c_void_p()
        if gguf_path is not None:
            rc = self._lib.vsl_engine_open(str(gguf_path).encode(), ctypes.byref(opt), ctypes.byref(h))
        else:
            s = make_spec(spec, init_std)
            rc = self._lib.vsl_engine_open_synthetic(ctypes.byref(s), seed, ctypes.byref(opt), ctypes.byref(h))
        check(rc, self._lib)
        self._h = h
        self.config = self.get_config()

    def close(self):
        if getattr(self, "_h", None):
            self._lib.vsl_engine_close(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def __enter__(self):
        return self

    def __exit__(self, *a):
        self.close()

    def get_config(self):
        s = ModelSpec()
        check(self._lib.vsl_engine_get_config(self._h, ctypes.byref(s)), self._lib)
        return {f: getattr(s, f) for f, _ in ModelSpec._fields_}

    def generate_ids(self, prompt, max_new, mode="greedy", temperature=0.0, top_k=40, seed=0, stop_on_eos=False,
                     return_logits=False, forced=None):
        """Token ids in, generated ids out (and each step's logits with return_logits).  forced: a
        token history of at least max_new - 1 ids; step t + 1 then takes forced[t] as its input
        instead of its own sample (teacher forcing; EOS does not stop the run)."""
        prompt = np.ascontiguousarray(prompt, dtype=np.uint32)
        p = GenParams(_MODES[mode] if isinstance(mode, str) else mode, temperature, top_k, int(bool(stop_on_eos)),
                      seed)
        out = np.zeros(max(max_new, 1), dtype=np.uint32)
        V = self.config["vocab_size"]
        logits = np.zeros((max(max_new, 1), V), dtype=np.float32) if return_logits else None
        n = ctypes.c_uint32(0)
        if forced is not None:
            f = np.ascontiguousarray(forced, dtype=np.uint32)
            check(self._lib.vsl_engine_generate_forced(self._h, _ptr(prompt), len(prompt), _ptr(f), len(f), max_new,
                                                       ctypes.byref(p), _ptr(out),
                                                       _ptr(logits) if return_logits else None, ctypes.byref(n)),
                  self._lib)
        else:
            check(self._lib.vsl_engine_generate_ids(self._h, _ptr(prompt), len(prompt), max_new, ctypes.byref(p),
                                                    _ptr(out), _ptr(logits) if return_logits else None,
                                                    ctypes.byref(n)), self._lib)
        toks = out[:n.value].copy()
        return (toks, logits[:n.value].copy()) if return_logits else toks

    def begin(self, prompt, max_new, mode="greedy", temperature=0.0, top_k=40, seed=0, stop_on_eos=False):
        prompt = np.ascontiguousarray(prompt, dtype=np.uint32)
        p = GenParams(_MODES[mode] if isinstance(mode, str) else mode, temperature, top_k, int(bool(stop_on_eos)),
                      seed)
        self._max_new = max_new
        check(self._lib.vsl_engine_begin(self._h, _ptr(prompt), len(prompt), max_new, ctypes.byref(p)), self._lib)

    def decode(self, n):
        issued = ctypes.c_uint32()
        check(self._lib.vsl_engine_decode(self._h, n, ctypes.byref(issued)), self._lib)
        return issued.value

    def sync(self):
        check(self._lib.vsl_engine_sync(self._h), self._lib)

    def finish(self):
        out = np.zeros(max(self._max_new, 1), dtype=np.uint32)
        n = ctypes.c_uint32()
        check(self._lib.vsl_engine_finish(self._h, _ptr(out), ctypes.byref(n)), self._lib)
        return out[:n.value].copy()

    def time_op(self, op, iterations=3):
        ms = ctypes.c_double()
        check(self._lib.vsl_engine_time_op(self._h, op, iterations, ctypes.byref(ms)), self._lib)
        return ms.value

    def generate(self, text, max_tokens=256, temperature=0.7, raw=False):
        """generate(): prompt + decode({id}) per generated token. Returns bytes when raw, else a str
        decoded as latin-1 (bytes kept 1:1, as the byte tokenizer emits them)."""
        b = text if isinstance(text, bytes) else text.encode()
        need = ctypes.c_uint64(0)
        cap = len(b) + 2 * max_tokens + 64
        for _ in range(2):  # a longer vocabulary text than the first guess: run again with its size
            buf = ctypes.create_string_buffer(cap)
            check(self._lib.vsl_engine_generate_text(self._h, b, max_tokens, temperature, buf, cap,
                                                     ctypes.byref(need)), self._lib)
            if need.value < cap:
                break
            cap = need.value + 1
        out = buf.raw[:need.value]
        return out if raw else out.decode("latin-1")

    def last_stats(self):
        s = GenStats()
        check(self._lib.vsl_engine_last_stats(self._h, ctypes.byref(s)), self._lib)
        return {f: getattr(s, f) for f, _ in GenStats._fields_ if f != "pad"}

    def vram_stats(self):
        s = PoolStats()
        check(self._lib.vsl_engine_vram_stats(self._h, ctypes.byref(s)), self._lib)
        return {f: getattr(s, f) for f, _ in PoolStats._fields_}

    def kv_bytes(self):
        v = ctypes.c_uint64()
        check(self._lib.vsl_engine_kv_bytes(self._h, ctypes.byref(v)), self._lib)
        return v.value

    def weight_bytes(self):
        v = ctypes.c_uint64()
        check(self._lib.vsl_engine_weight_bytes(self._h, ctypes.byref(v)), self._lib)
        return v.value

    def benchmark(self, warmup=10, tokens=100, iterations=3):
        a, lo, hi = ctypes.c_double(), ctypes.c_double(), ctypes.c_double()
        check(self._lib.vsl_engine_benchmark(self._h, warmup, tokens, iterations, ctypes.byref(a), ctypes.byref(lo),
                                             ctypes.byref(hi)), self._lib)
        return a.value, lo.value, hi.value

    def packs(self):
        """Resident packs: [{name, type, layer_idx, priority, bytes, dtype, tier, device_ptr, ...}]."""
        n = _U64()
        check(self._lib.vsl_engine_pack_count(self._h, ctypes.byref(n)), self._lib)
        out = []
        for i in range(n.value):
            info, name = PackInfo(), ctypes.create_string_buffer(256)
            check(self._lib.vsl_engine_pack(self._h, i, ctypes.byref(info), name, 256), self._lib)
            d = {f: getattr(info, f) for f, _ in PackInfo._fields_}
            d["name"] = name.value.decode()
            out.append(d)
        return out

    def read_tensor(self, name, nbytes):
        buf = np.empty(nbytes, dtype=np.uint8)
        dt = ctypes.c_int()
        check(self._lib.vsl_engine_read_tensor(self._h, name.encode(), _ptr(buf), nbytes, ctypes.byref(dt)),
              self._lib)
        return buf.view(np.float16 if dt.value == VSL_DT_F16 else np.float32)
