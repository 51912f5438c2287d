#!/usr/bin/env python3
"""Decode throughput (tok/s, HBM GB/s and fraction of peak) and prefill throughput of the 8B-class
fp16 Llama-style decoder at batch 1 on one MI355X, through the engine's C ABI.

Workload: 32 layers, d_model 4096, 32 query / 8 KV heads (head_dim 128), SwiGLU FFN 14336, vocab
32000, RMSNorm eps 1e-5, RoPE theta 500000, fp16 weights N(0, 0.02) generated on the device, KV
cache fp16 with capacity 4096; prompt of 512 uniform-random token ids (prefill timed on its own),
then greedy decode.  A step is one decode token; K steps are timed between two synchronisations.

The same run also measures, as extra keys of the one JSON line: the configured 512-step decode
(positions 513..1024), the 1B-class model (prompt 128, greedy decode 256), the fp16 GEMV sweep, the
long-context workload (8192-token prompt in 2048-token chunks, KV capacity 32768), a 70B-class model
(137.5 GB of fp16 weights in one GPU's HBM; prompt 128, greedy decode 64; again with Q4_0 weight
blocks read by the decode) and the 8B-class model with Q8_0 / Q4_0 weight blocks read by the decode
(prompt 512, greedy decode 128); --quick skips them.

Prints one JSON line.  --gpus N with N > 1 exits: this build targets one GPU.
"""
import argparse
import importlib.util
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
PEAK_HBM = 8.0e12       # MI355X HBM3E, bytes/s
PEAK_F16 = 2.5e15       # MI355X dense fp16 MFMA, flop/s

CFG = dict(hidden_size=4096, num_layers=32, num_heads=32, num_kv_heads=8, intermediate_size=14336, vocab_size=32000,
           max_position_embeddings=32768, rope_theta=500000.0, rms_eps=1e-5, dtype=1)
KV_CAPACITY = 4096

LLAMA_1B = dict(hidden_size=2048, num_layers=16, num_heads=32, num_kv_heads=8, intermediate_size=8192,
                vocab_size=32000, max_position_embeddings=4096, rope_theta=10000.0, rms_eps=1e-5, dtype=1)

# The rocprofv3 summary whose FETCH_SIZE / WRITE_SIZE columns give the dominant decode kernel's HBM
# traffic per launch (counters scaled by a copy kernel of known size, as the file states).
PROFILE = os.path.join(ROOT, "profiles", "llama8b_decode_prefill_rocprof.md")
DOMINANT_KERNEL_ROW = "`k_gemv_dec<WF16, 2, 4, 2, WF32, 4, 4>`"


def profiled_traffic(path=PROFILE, row=DOMINANT_KERNEL_ROW):
    """HBM bytes per launch (FETCH + WRITE, MB = 1e6 bytes) of the dominant decode kernel, read from
    the kernel table of the committed profile summary; None when the row is missing."""
    try:
        with open(path) as f:
            for line in f:
                if line.startswith("| " + row):
                    cols = [c.strip() for c in line.strip().strip("|").split("|")]
                    return int(round((float(cols[5]) + float(cols[6])) * 1e6))
    except (OSError, ValueError, IndexError):
        return None
    return None


def host_facts():
    """CPU model, sockets / NUMA nodes of the host, and the CPUs and memory nodes this process may use."""
    import subprocess
    facts = {"cpus_allowed": len(os.sched_getaffinity(0)), "nproc": os.cpu_count()}
    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
        for line in out.splitlines():
            k, _, v = line.partition(":")
            k, v = k.strip(), v.strip()
            if k in ("Model name", "Socket(s)", "NUMA node(s)", "Thread(s) per core", "Core(s) per socket"):
                facts[k.lower().replace("(s)", "s").replace(" ", "_")] = v
    except Exception:
        pass
    try:
        with open("/proc/self/status") as f:
            for line in f:
                if line.startswith(("Cpus_allowed_list", "Mems_allowed_list")):
                    k, _, v = line.partition(":")
                    facts[k.strip().lower()] = v.strip()
    except OSError:
        pass
    return facts


def load_package():
    name = "vulkan_symbiote_loader_amd"
    spec = importlib.util.spec_from_file_location(name, os.path.join(ROOT, "vulkan-symbiote-loader_amd", "__init__.py"))
    mod = importlib.util.module_from_spec(spec)
    sys.modules[name] = mod
    spec.loader.exec_module(mod)
    return mod


def model_bytes(c):
    d, L, nq, nkv, F, V = (c["hidden_size"], c["num_layers"], c["num_heads"], c["num_kv_heads"],
                           c["intermediate_size"], c["vocab_size"])
    hd = d // nq
    p_lin = L * (d * nq * hd + 2 * d * nkv * hd + nq * hd * d + 3 * d * F) + V * d
    p_norm = L * 2 * d + d
    kvb = 2 * L * nkv * hd * 2  # K and V, fp16, per position
    return p_lin, p_norm, kvb


# bytes per linear weight read by the decode, by the model's weight storage (VSL_WF_*): fp32, fp16, and
# the resident block-quantized packs (values plus one fp32 scale per 32 weights; Q4_1 also an offset)
WEIGHT_BYTES = {0: 4.0, 1: 2.0, 2: 0.5 + 4 / 32, 3: 0.5 + 8 / 32, 4: 1.0 + 4 / 32}


def decode_bytes(c, attended):
    """Algorithmic HBM bytes of one decode token that attends `attended` positions: every weight
    once, the embedding row, K/V of the attended positions and the new position's K/V write."""
    p_lin, p_norm, kvb = model_bytes(c)
    return WEIGHT_BYTES[c.get("dtype", 1)] * p_lin + 2 * p_norm + 2 * c["hidden_size"] + kvb * attended + kvb


def prefill_flops(c, S):
    d, L, nq, V = c["hidden_size"], c["num_layers"], c["num_heads"], c["vocab_size"]
    hd = d // nq
    p_lin, _, _ = model_bytes(c)
    p_layers = p_lin - V * d
    return 2 * S * p_layers + 2 * V * d + 4 * L * nq * hd * S * (S + 1) / 2


def cpu_baseline(eng, cfg, prompt, seconds):
    """The oracle (CPU restatement of the reference's token loop) on this host, timed on a bounded
    sample of the same workload: the engine's resident weights copied to host memory, the bench's
    prompt processed (untimed), then greedy decode steps from the next position for about `seconds`."""
    sys.path.insert(0, ROOT)
    from oracle import oracle as orc
    d, L, nq, nkv, F, V = (cfg["hidden_size"], cfg["num_layers"], cfg["num_heads"], cfg["num_kv_heads"],
                           cfg["intermediate_size"], cfg["vocab_size"])
    hd = d // nq
    m = orc.Model(config=dict(hidden_size=d, num_layers=L, num_heads=nq, num_kv_heads=nkv, intermediate_size=F,
                              vocab_size=V, head_dim=hd, max_position_embeddings=cfg["max_position_embeddings"],
                              rope_theta=cfg["rope_theta"], rms_eps=cfg["rms_eps"]))
    sizes = {"token_embd.weight": V * d, "output.weight": V * d}
    for l in range(L):
        sizes.update({f"blk.{l}.attn_q.weight": nq * hd * d, f"blk.{l}.attn_k.weight": nkv * hd * d,
                      f"blk.{l}.attn_v.weight": nkv * hd * d, f"blk.{l}.attn_o.weight": d * nq * hd,
                      f"blk.{l}.ffn_gate.weight": F * d, f"blk.{l}.ffn_up.weight": F * d,
                      f"blk.{l}.ffn_down.weight": d * F})
    for n, cnt in sizes.items():
        m.set_tensor(n, eng.read_tensor(n, cnt * 2))
    for n in ["output_norm.weight"] + [f"blk.{l}.{s}.weight" for l in range(L) for s in ("attn_norm", "ffn_norm")]:
        m.set_tensor(n, eng.read_tensor(n, d * 4))
    threads = orc.num_threads()
    t0 = time.perf_counter()
    n, secs = m.decode_rate(prompt, max_seconds=seconds, max_tokens=4096)
    wall = time.perf_counter() - t0
    m.close()
    return {"value": n / secs, "unit": "tok/s", "cores": threads, "kind": "port",
            "sample": f"oracle greedy decode of {n} tokens at positions {len(prompt) + 1}..{len(prompt) + n} after "
                      f"the bench's {len(prompt)}-token prompt (processed untimed, {wall - secs:.1f} s) on the same "
                      f"8B weights ({secs:.1f} s timed, {threads} OpenMP threads, fp16 weights / fp32 math)",
            "host": host_facts()}


def gpus_or_exit(a):
    if a.gpus != 1:
        print(f"bench.py: this build runs on one GPU; --gpus {a.gpus} is not supported (use --gpus 1)",
              file=sys.stderr)
        sys.exit(2)


def sweep_leg(vsl, graph=True):
    """GEMV sweep: W [N,K] fp16 ~N(0,0.02), X [K,B] fp16 ~N(0,1), fp32 accumulate, fp16 Y; W rotated
    over >= 512 MB of distinct copies so the 256 MB MALL cannot serve it.  Each point times >= 64
    launches back to back: captured in one hipGraph and replayed (graph=True, as the decode step runs
    its kernels; a Python loop of launches cannot issue a 5 us kernel as fast as the GPU retires it),
    or launched one by one (graph=False: what rocprofv3's kernel trace follows).  Returns the per-shape
    rows and geometric means (all shapes, and per B)."""
    import ctypes
    H = vsl.hip()
    P = ctypes.c_void_p
    arena = P()
    vsl.check(H.vsl_arena_create(0, 1 << 30, ctypes.byref(arena)))

    def alloc(n):
        p = P()
        vsl.check(H.vsl_arena_alloc(arena, n, 256, ctypes.byref(p)))
        return p

    rot_bytes = 512 << 20
    wmax = 32000 * 4096 * 2
    ncopy = -(-rot_bytes // wmax) + 1
    wbuf = alloc(ncopy * wmax if ncopy * wmax >= rot_bytes else rot_bytes + wmax)
    wtotal = max(ncopy * wmax, rot_bytes + wmax)
    vsl.check(H.vsl_fill_normal(wbuf, vsl.VSL_DT_F16, wtotal // 2, 1, b"sweep.W", 0.0, 0.02, None))
    xbuf = alloc(14336 * 16 * 2)
    vsl.check(H.vsl_fill_normal(xbuf, vsl.VSL_DT_F16, 14336 * 16, 2, b"sweep.X", 0.0, 1.0, None))
    ybuf = alloc(32000 * 16 * 2)
    e0, e1, stream = P(), P(), P()
    vsl.check(H.vsl_event_create(ctypes.byref(e0)))
    vsl.check(H.vsl_event_create(ctypes.byref(e1)))
    vsl.check(H.vsl_stream_create(ctypes.byref(stream)))
    rows = []
    for (N, K) in [(4096, 4096), (14336, 4096), (4096, 14336), (32000, 4096)]:
        wsz = N * K * 2
        copies = max(2, -(-rot_bytes // wsz))
        ptrs = [P(wbuf.value + (i * wsz) % (wtotal - wsz)) for i in range(copies)]
        for B in (1, 4, 16):
            # X as B contiguous K-vectors (vsl_gemv_batched); Y [B][N] fp16
            args = lambda w: (w, N, K, xbuf, B, ybuf, vsl.VSL_DT_F16, stream)
            for w in ptrs[:2]:
                vsl.check(H.vsl_gemv_batched(*args(w)))
            reps = max(copies * 4, 64)
            g = P()
            if graph:
                vsl.check(H.vsl_graph_begin(stream))
                for i in range(reps):
                    vsl.check(H.vsl_gemv_batched(*args(ptrs[i % copies])))
                vsl.check(H.vsl_graph_end(stream, ctypes.byref(g)))
                vsl.check(H.vsl_graph_launch(g, stream))  # one untimed replay
            vsl.check(H.vsl_stream_sync(stream))
            vsl.check(H.vsl_event_record(e0, stream))
            if graph:
                vsl.check(H.vsl_graph_launch(g, stream))
            else:
                for i in range(reps):
                    vsl.check(H.vsl_gemv_batched(*args(ptrs[i % copies])))
            vsl.check(H.vsl_event_record(e1, stream))
            vsl.check(H.vsl_event_sync(e1))
            if graph:
                vsl.check(H.vsl_graph_destroy(g))
            ms = ctypes.c_float()
            vsl.check(H.vsl_event_elapsed_ms(e0, e1, ctypes.byref(ms)))
            us = ms.value * 1e3 / reps
            nbytes = 2 * N * K + 2 * K * B + 2 * N * B
            rows.append({"N": N, "K": K, "B": B, "us": round(us, 2), "gbps": round(nbytes / us / 1e3, 1),
                         "hbm_frac": round(nbytes / us / 1e3 / (PEAK_HBM / 1e9), 4),
                         "tflops": round(2 * N * K * B / us / 1e6, 2)})
    vsl.check(H.vsl_event_destroy(e0))
    vsl.check(H.vsl_event_destroy(e1))
    vsl.check(H.vsl_stream_destroy(stream))
    vsl.check(H.vsl_arena_destroy(arena))
    geo = lambda rs: round(float(np.exp(np.mean([np.log(r["gbps"]) for r in rs]))), 1)
    return {"geomean_gbps": geo(rows), "geomean_hbm_frac": round(geo(rows) / (PEAK_HBM / 1e9), 4),
            "geomean_gbps_by_B": {str(B): geo([r for r in rows if r["B"] == B]) for B in (1, 4, 16)},
            "shapes": rows}


def run_sweep(a):
    gpus_or_exit(a)
    sw = sweep_leg(load_package(), graph=not a.eager)
    out = {"metric": "GEMV sweep HBM GB/s (geometric mean over 12 shapes), fp16 W/X/Y, fp32 accumulate",
           "value": sw["geomean_gbps"], "unit": "GB/s", "n_gpus": 1, "higher_is_better": True, "dtype": "f16",
           "data": "synthetic: W ~N(0,0.02), X ~N(0,1) fp16 (Philox on device); W rotated over >= 512 MB",
           "config": {"workload": "GEMV / skinny-GEMM sweep y = W X, (N,K) in {(4096,4096),(14336,4096),"
                                  "(4096,14336),(32000,4096)}, B in {1,4,16}"}}
    out.update(sw)
    print(json.dumps(out), flush=True)


def timed_decode(eng, prompt, steps, **kw):
    """One generation: the prompt pass, then exactly `steps` decode steps between two synchronisations.
    Returns (decode seconds, the engine's stats of the generation)."""
    eng.begin(prompt, steps + 1, **kw)
    eng.sync()
    t0 = time.perf_counter()
    issued = eng.decode(steps)
    eng.sync()
    dt = time.perf_counter() - t0
    toks = eng.finish()
    assert issued == steps and len(toks) == steps + 1, (issued, len(toks))
    return dt, eng.last_stats()


def decode_rates(cfg, n_prompt, steps, secs):
    """tok/s and algorithmic HBM rate of `steps` decode steps after an n_prompt-token prompt (step i
    processes position n_prompt + i - 1 and attends n_prompt + i positions)."""
    total = sum(decode_bytes(cfg, n_prompt + i) for i in range(1, steps + 1))
    return {"tok_s": round(steps / secs, 2), "ms_per_step": round(secs * 1e3 / steps, 4),
            "hbm_gbps": round(total / secs / 1e9, 1), "hbm_frac": round(total / secs / PEAK_HBM, 4),
            "bytes_per_token": int(total / steps)}


def long_leg(vsl, steps, eager):
    """Long-context workload: 8B-class fp16, prompt 8192 prefilled in 2048-row chunks, KV capacity 32768,
    greedy decode, the same decode with T=0.7 top-k 40 seeded sampling, and with the windowed mode at
    the reference's parameters (window 512, 16 global tokens, from sequence length 8193 on)."""
    n_prompt, cap, chunk = 8192, 32768, 2048
    prompt = np.random.default_rng(1).integers(0, CFG["vocab_size"], n_prompt).astype(np.uint32)
    eng = vsl.Engine(spec=CFG, seed=0, kv_capacity=cap, prefill_chunk=chunk, use_graph=not eager)
    try:
        eng.begin(prompt, 3)  # warmup: capture, caches
        eng.decode(2)
        eng.finish()
        dec_s, st = timed_decode(eng, prompt, steps)
        samp_s, _ = timed_decode(eng, prompt, steps, mode="topk", temperature=0.7, top_k=40, seed=7)
    finally:
        eng.close()
    pre_s = st["prefill_ms"] / 1e3
    pre_flops = prefill_flops(CFG, n_prompt)
    out = {"workload": f"8B-class fp16 bs=1: prompt {n_prompt} prefilled in {chunk}-token chunks, KV cap {cap}, "
                       f"decode {steps} greedy, then {steps} with T=0.7 top-k 40 seeded sampling",
           "decode": decode_rates(CFG, n_prompt, steps, dec_s),
           "sampled_tok_s": round(steps / samp_s, 2),
           "prefill_tok_s": round(n_prompt / pre_s, 1), "prefill_ms": round(st["prefill_ms"], 3),
           "prefill_tflops": round(pre_flops / pre_s / 1e12, 1),
           "prefill_mfma_frac": round(pre_flops / pre_s / PEAK_F16, 4)}
    win = (512, 16, 8192)
    eng = vsl.Engine(spec=CFG, seed=0, kv_capacity=cap, prefill_chunk=chunk, use_graph=not eager, window=win)
    try:
        eng.begin(prompt, 3)
        eng.decode(2)
        eng.finish()
        win_s, _ = timed_decode(eng, prompt, steps)
    finally:
        eng.close()
    n_att = win[1] + win[0] + 1
    win_bytes = sum(decode_bytes(CFG, n_prompt + i if n_prompt + i <= win[2] else n_att) for i in range(1, steps + 1))
    out["window"] = {"sparse_window": win[0], "sparse_global": win[1], "sparse_threshold": win[2],
                     "decode_tok_s": round(steps / win_s, 2), "hbm_gbps": round(win_bytes / win_s / 1e9, 1),
                     "hbm_frac": round(win_bytes / win_s / PEAK_HBM, 4)}
    return out


def run_long(a):
    gpus_or_exit(a)
    steps = a.steps if a.steps != 512 else 128
    lg = long_leg(load_package(), steps, a.eager)
    out = {
        "metric": "decode tok/s + HBM GB/s (% peak), 8B fp16 bs=1, long context; prefill tok/s",
        "value": lg["decode"]["tok_s"], "unit": "tok/s", "n_gpus": 1, "steps": steps, "warmup": 2,
        "ms_per_step": lg["decode"]["ms_per_step"], "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "f16",
        "data": "synthetic: random-init N(0,0.02) fp16 weights (Philox on device), uniform-random prompt ids",
        "config": {"workload": lg["workload"], "global_batch": 1, "seq_len": 8192 + steps,
                   "parallelism": "single-gpu"},
        "decode_launch": "eager" if a.eager else "hipGraph replay",
    }
    out.update(lg)
    print(json.dumps(out), flush=True)


def decode_ops_table(eng, cfg, p_att, iterations=3):
    """Each decode op's average device time per launch (HIP events on the engine's stream, every layer
    visited per round, so no weight is served from the MALL) with its algorithmic bytes and rate."""
    d, F, V = cfg["hidden_size"], cfg["intermediate_size"], cfg["vocab_size"]
    nq, nkv = cfg["num_heads"], cfg["num_kv_heads"]
    hd = d // nq
    wb = WEIGHT_BYTES[cfg.get("dtype", 1)]  # bytes per linear weight
    names = ["qkv_rope_append", "attn_decode", "o_proj_resid", "norm_gateup_swiglu", "down_proj_resid",
             "lm_head_argmax"]
    bytes_per_launch = [
        wb * (nq + 2 * nkv) * hd * d + 8 * d + 4 * nq * hd + 2 * 2 * nkv * hd,
        2 * 2 * nkv * hd * p_att + 8 * nq * hd,
        wb * d * nq * hd + 4 * nq * hd + 8 * d,
        wb * 2 * F * d + 8 * d + 4 * F,
        wb * d * F + 4 * F + 8 * d,
        wb * V * d + 8 * d + 4 * V,
    ]
    ops = {}
    for op, nm in enumerate(names):
        ms = eng.time_op(op, iterations)
        ops[nm] = {"avg_us": round(ms * 1e3, 2), "bytes": int(bytes_per_launch[op]),
                   "gbps": round(bytes_per_launch[op] / (ms * 1e-3) / 1e9, 1)}
    return ops


def llama_1b_leg(vsl, eager, prefill_runs=5, kernel_timing=True, steps=256):
    """1B-class fp16 (16 layers, d 2048, 32/8 heads, FFN 8192, V 32000): prompt 128, greedy decode 256
    (`steps` shortens the decode for profiling runs)."""
    n_prompt = 128
    prompt = np.random.default_rng(2).integers(0, LLAMA_1B["vocab_size"], n_prompt).astype(np.uint32)
    eng = vsl.Engine(spec=LLAMA_1B, seed=0, kv_capacity=1024, use_graph=not eager)
    try:
        eng.begin(prompt, 9)
        eng.decode(8)
        eng.finish()
        dec_s, st = timed_decode(eng, prompt, steps)
        pre = [st["prefill_ms"]]
        for _ in range(prefill_runs - 1):
            eng.begin(prompt, 1)
            eng.finish()
            pre.append(eng.last_stats()["prefill_ms"])
        # per-op times at the decode's last position (the KV length of the final step)
        ops = decode_ops_table(eng, LLAMA_1B, n_prompt + steps) if kernel_timing else None
    finally:
        eng.close()
    pre_ms = float(np.median(pre))
    pre_flops = prefill_flops(LLAMA_1B, n_prompt)
    out = {"workload": f"1B-class Llama decoder fp16 bs=1 (16L, d2048, 32/8 heads, FFN 8192, V32000): prompt "
                       f"{n_prompt}, greedy decode {steps}",
           "decode": decode_rates(LLAMA_1B, n_prompt, steps, dec_s),
           "prefill_ms": round(pre_ms, 3), "prefill_tok_s": round(n_prompt / (pre_ms / 1e3), 1),
           "prefill_tflops": round(pre_flops / (pre_ms / 1e3) / 1e12, 1),
           "prefill_mfma_frac": round(pre_flops / (pre_ms / 1e3) / PEAK_F16, 4)}
    if ops is not None:
        out["decode_ops"] = ops
    return out


# A 70B-class decoder (Llama-2/3-70B geometry: 80 layers, d 8192, 64/8 heads, FFN 28672), fp16: 137.5 GB
# of weights, which one MI355X holds in its 288 GB of HBM.
LLAMA_70B = dict(hidden_size=8192, num_layers=80, num_heads=64, num_kv_heads=8, intermediate_size=28672,
                 vocab_size=32000, max_position_embeddings=4096, rope_theta=500000.0, rms_eps=1e-5, dtype=1)


def llama_70b_leg(vsl, eager, steps=64, prefill_runs=3, fmt=1):
    """70B-class on one GPU: prompt 128, greedy decode `steps`; fmt 1 fp16 weights, or VSL_WF_Q4_0 /
    Q4_1 / Q8_0: every linear weight quantized on the device into resident blocks for the decode (the
    prompt pass on the expanded fp16 packs)."""
    n_prompt = 128
    cfg = dict(LLAMA_70B, dtype=fmt)
    prompt = np.random.default_rng(3).integers(0, LLAMA_70B["vocab_size"], n_prompt).astype(np.uint32)
    eng = vsl.Engine(spec=cfg, seed=0, kv_capacity=1024, use_graph=not eager)
    try:
        eng.begin(prompt, 5)
        eng.decode(4)
        eng.finish()
        dec_s, st = timed_decode(eng, prompt, steps)
        pre = [st["prefill_ms"]]
        for _ in range(prefill_runs - 1):
            eng.begin(prompt, 1)
            eng.finish()
            pre.append(eng.last_stats()["prefill_ms"])
    finally:
        eng.close()
    pre_ms = float(np.median(pre))
    pre_flops = prefill_flops(LLAMA_70B, n_prompt)
    name = {1: "fp16", vsl.VSL_WF_Q8_0: "Q8_0 resident blocks", vsl.VSL_WF_Q4_0: "Q4_0 resident blocks",
            vsl.VSL_WF_Q4_1: "Q4_1 resident blocks"}[fmt]
    wgb = decode_bytes(cfg, 0) / 1e9
    return {"workload": f"70B-class Llama decoder {name} bs=1 (80L, d8192, 64/8 heads, FFN 28672, V32000; "
                        f"{wgb:.1f} GB read per token on one GPU): prompt {n_prompt}, greedy decode {steps}",
            "decode": decode_rates(cfg, n_prompt, steps, dec_s),
            "prefill_ms": round(pre_ms, 3), "prefill_tok_s": round(n_prompt / (pre_ms / 1e3), 1),
            "prefill_tflops": round(pre_flops / (pre_ms / 1e3) / 1e12, 1),
            "prefill_mfma_frac": round(pre_flops / (pre_ms / 1e3) / PEAK_F16, 4)}


def llama_8b_quant_leg(vsl, fmt, eager, steps=128, prefill_runs=3, kernel_timing=False):
    """The 8B-class model with every linear weight block-quantized (VSL_WF_Q8_0 / Q4_0 / Q4_1, quantized
    on the device from the fp16 draws): the decode GEMVs read the resident blocks, the prompt pass runs
    on the expanded fp16 packs. Prompt 512, greedy decode `steps`; with kernel_timing also the per-op
    table at the last decode position."""
    cfg = dict(CFG, dtype=fmt)
    prompt = np.random.default_rng(1).integers(0, cfg["vocab_size"], 512).astype(np.uint32)
    eng = vsl.Engine(spec=cfg, seed=0, kv_capacity=KV_CAPACITY, use_graph=not eager)
    try:
        eng.begin(prompt, 9)
        eng.decode(8)
        eng.finish()
        dec_s, st = timed_decode(eng, prompt, steps)
        pre = [st["prefill_ms"]]
        for _ in range(prefill_runs - 1):
            eng.begin(prompt, 1)
            eng.finish()
            pre.append(eng.last_stats()["prefill_ms"])
        ops = decode_ops_table(eng, cfg, 512 + steps) if kernel_timing else None
    finally:
        eng.close()
    name = {vsl.VSL_WF_Q8_0: "Q8_0", vsl.VSL_WF_Q4_0: "Q4_0", vsl.VSL_WF_Q4_1: "Q4_1"}[fmt]
    out = {"workload": f"8B-class Llama decoder, linear weights {name} resident blocks (quantized on the device "
                       f"from N(0, 0.02) fp16 draws), bs=1: prompt 512, greedy decode {steps}, KV cap {KV_CAPACITY}",
           "decode": decode_rates(cfg, 512, steps, dec_s),
           "prefill_ms": round(float(np.median(pre)), 3)}
    if ops is not None:
        out["decode_ops"] = ops
    return out


def copy_calibration(vsl, mb):
    """One device-to-device copy of `mb` MiB: a kernel of known traffic for scaling rocprofv3's
    FETCH_SIZE / WRITE_SIZE counters. Returns the bytes copied."""
    import ctypes
    H = vsl.hip()
    nbytes = mb << 20
    arena = ctypes.c_void_p()
    vsl.check(H.vsl_arena_create(0, 2 * nbytes + (1 << 20), ctypes.byref(arena)))
    src, dst = ctypes.c_void_p(), ctypes.c_void_p()
    vsl.check(H.vsl_arena_alloc(arena, nbytes, 256, ctypes.byref(src)))
    vsl.check(H.vsl_arena_alloc(arena, nbytes, 256, ctypes.byref(dst)))
    vsl.check(H.vsl_copy_d2d(dst, src, nbytes, None))
    vsl.check(H.vsl_device_sync())
    vsl.check(H.vsl_arena_destroy(arena))
    return nbytes


def main():
    ap = argparse.ArgumentParser(description=__doc__)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=512, help="timed decode steps (tokens)")
    ap.add_argument("--warmup", type=int, default=32, help="untimed decode steps before the timed run")
    ap.add_argument("--prompt", type=int, default=512)
    ap.add_argument("--prefill-runs", type=int, default=5, help="prompt passes timed; the median is reported")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=15.0)
    ap.add_argument("--llama-1b", action="store_true",
                    help="the 1B-class workload alone (prompt 128, greedy decode 256): one JSON line")
    ap.add_argument("--steps-1b", type=int, default=256,
                    help="decode steps of the 1B-class workload (256 as configured; fewer for profiling runs)")
    ap.add_argument("--attn-splits", type=int, default=0,
                    help="decode attention split count of the 8B engine (0: the engine's choice)")
    ap.add_argument("--quick", action="store_true",
                    help="the headline decode / prefill only (no 512-step decode, 1B, sweep, long-context, 70B "
                         "or quantized legs)")
    ap.add_argument("--no-kernel-timing", action="store_true")
    ap.add_argument("--copy-calibration-mb", type=int, default=0,
                    help="after the run, copy this many MB device-to-device once (a kernel of known traffic "
                         "for scaling rocprofv3 FETCH_SIZE / WRITE_SIZE counters)")
    ap.add_argument("--eager", action="store_true",
                    help="launch each decode step's kernels (and each GEMV sweep launch) directly instead of "
                         "replaying a captured hipGraph (same kernels; used under rocprofv3, whose graph-launch "
                         "interception crashes here)")
    ap.add_argument("--sweep", action="store_true",
                    help="the standalone fp16 GEMV / skinny-GEMM sweep instead: Y = W X for (N, K) in "
                         "{(4096,4096), (14336,4096), (4096,14336), (32000,4096)} and B in {1, 4, 16}, W rotated "
                         "over >= 512 MB of distinct copies so the 256 MB MALL cannot serve it")
    ap.add_argument("--quant", choices=["q8_0", "q4_0", "q4_1"],
                    help="the 8B-class model with block-quantized linear weights alone (resident blocks read "
                         "by the decode; prompt 512, greedy decode 128) with its per-op table: one JSON line")
    ap.add_argument("--long", action="store_true",
                    help="the long-context workload instead: 8192-token prompt prefilled in 2048-token chunks "
                         "into a 32768-position KV cache, greedy decode (default 128 steps), then the same "
                         "decode with T=0.7 top-k 40 seeded sampling")
    a = ap.parse_args()
    if a.long:
        run_long(a)
        return
    if a.sweep:
        run_sweep(a)
        return
    if a.quant:
        gpus_or_exit(a)
        vsl = load_package()
        fmt = {"q8_0": vsl.VSL_WF_Q8_0, "q4_0": vsl.VSL_WF_Q4_0, "q4_1": vsl.VSL_WF_Q4_1}[a.quant]
        lg = llama_8b_quant_leg(vsl, fmt, a.eager, kernel_timing=not a.no_kernel_timing)
        out = {"metric": f"decode tok/s + HBM GB/s (% peak), 8B {a.quant.upper()} bs=1; prefill ms",
               "value": lg["decode"]["tok_s"], "unit": "tok/s", "n_gpus": 1, "higher_is_better": True,
               "dtype": a.quant, "data": "synthetic: N(0,0.02) fp16 draws quantized on the device, uniform-random "
                                         "prompt ids", "config": {"workload": lg["workload"]}}
        out.update(lg)
        print(json.dumps(out), flush=True)
        return
    if a.llama_1b:
        gpus_or_exit(a)
        vsl = load_package()
        lg = llama_1b_leg(vsl, a.eager, kernel_timing=not a.no_kernel_timing, steps=a.steps_1b)
        out = {"metric": "decode tok/s + HBM GB/s (% peak), 1B fp16 bs=1; prefill tok/s",
               "value": lg["decode"]["tok_s"], "unit": "tok/s", "n_gpus": 1, "higher_is_better": True,
               "dtype": "f16", "data": "synthetic: random-init N(0,0.02) fp16 weights, uniform-random prompt ids",
               "config": {"workload": lg["workload"]}}
        out.update(lg)
        if a.copy_calibration_mb:
            out["copy_calibration_bytes"] = copy_calibration(vsl, a.copy_calibration_mb)
        print(json.dumps(out), flush=True)
        return
    gpus_or_exit(a)
    if a.prompt + a.steps > KV_CAPACITY:
        print("bench.py: prompt + steps exceed the KV capacity", file=sys.stderr)
        sys.exit(2)

    vsl = load_package()
    t_init = time.perf_counter()
    eng = vsl.Engine(spec=CFG, seed=0, kv_capacity=KV_CAPACITY, use_graph=not a.eager, attn_splits=a.attn_splits)
    init_s = time.perf_counter() - t_init
    prompt = np.random.default_rng(1).integers(0, CFG["vocab_size"], a.prompt).astype(np.uint32)

    # warmup: one full generation (graph capture, caches, clocks)
    eng.begin(prompt, a.warmup + 1)
    eng.decode(a.warmup)
    eng.finish()

    # timed: prefill (events) + exactly K decode steps between two synchronisations
    eng.begin(prompt, a.steps + 1)
    eng.sync()
    t0 = time.perf_counter()
    issued = eng.decode(a.steps)
    eng.sync()
    t1 = time.perf_counter()
    toks = eng.finish()
    st = eng.last_stats()
    assert issued == a.steps and len(toks) == a.steps + 1, (issued, len(toks))
    dec_s = t1 - t0
    tok_s = a.steps / dec_s
    # prefill: the median of several prompt passes (each one generation of a single token)
    pre_runs = [st["prefill_ms"]]
    for _ in range(a.prefill_runs - 1):
        eng.begin(prompt, 1)
        eng.finish()
        pre_runs.append(eng.last_stats()["prefill_ms"])
    pre_ms = float(np.median(pre_runs))
    # step i (1..K) processes position prompt+i-1 and attends prompt+i positions
    total_bytes = sum(decode_bytes(CFG, a.prompt + i) for i in range(1, a.steps + 1))
    hbm = total_bytes / dec_s
    pre_s = pre_ms / 1e3
    pre_flops = prefill_flops(CFG, a.prompt)

    out = {
        "metric": "decode tok/s + HBM GB/s (% peak), 8B fp16 bs=1; prefill tok/s",
        "value": round(tok_s, 2),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": a.steps,
        "warmup": a.warmup,
        "ms_per_step": round(dec_s * 1e3 / a.steps, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16",
        "data": "synthetic: random-init N(0,0.02) fp16 weights (Philox on device), uniform-random prompt ids",
        "config": {"workload": f"8B-class Llama decoder fp16 bs=1 (32L, d4096, 32/8 heads, FFN 14336, V32000): "
                               f"prompt {a.prompt}, greedy decode {a.steps}, KV cap {KV_CAPACITY}",
                   "global_batch": 1, "seq_len": a.prompt + a.steps, "parallelism": "single-gpu"},
        "decode_hbm_gbps": round(hbm / 1e9, 1),
        "decode_hbm_frac": round(hbm / PEAK_HBM, 4),
        "decode_bytes_per_token": int(total_bytes / a.steps),
        "decode_ms_events": round(st["decode_ms"], 3),
        "prefill_tok_s": round(a.prompt / pre_s, 1),
        "prefill_ms": round(pre_ms, 3),
        "prefill_runs_ms": [round(x, 3) for x in pre_runs],
        "prefill_tflops": round(pre_flops / pre_s / 1e12, 1),
        "prefill_mfma_frac": round(pre_flops / pre_s / PEAK_F16, 4),
        "engine_init_s": round(init_s, 2),
        "decode_launch": "eager" if a.eager else "hipGraph replay",
    }

    if not a.no_kernel_timing:
        ops = decode_ops_table(eng, CFG, a.prompt + a.steps)
        dom = ops["norm_gateup_swiglu"]
        achieved = dom["bytes"] / (dom["avg_us"] * 1e-6)
        out["roofline"] = {"bound": "hbm", "achieved": round(achieved / 1e9, 1), "peak": 8000.0, "unit": "GB/s",
                           "frac": round(achieved / PEAK_HBM, 4), "traffic": profiled_traffic(),
                           "algorithmic_bytes": dom["bytes"],
                           "kernel": "k_gemv_dec<EPI_SWIGLU> (ffn norm + [Wgate;Wup] GEMV + SwiGLU)",
                           "traffic_source": os.path.relpath(PROFILE, ROOT) + " (FETCH_SIZE + WRITE_SIZE columns "
                                             "of the kernel's row, read at run time)"}
        out["decode_ops"] = ops

    # the configured decode length: 512 greedy steps after the 512-token prompt (positions 513..1024)
    if not a.quick and a.prompt + 512 <= KV_CAPACITY:
        secs, _ = timed_decode(eng, prompt, 512)
        out["decode_512"] = dict(decode_rates(CFG, a.prompt, 512, secs),
                                 workload=f"prompt {a.prompt}, greedy decode 512 (positions {a.prompt + 1}.."
                                          f"{a.prompt + 512}), KV cap {KV_CAPACITY}")

    if not a.no_cpu_baseline:
        try:
            out["cpu_baseline"] = cpu_baseline(eng, CFG, prompt, a.cpu_seconds)
        except Exception as ex:  # reported, never fatal to the GPU measurement
            out["cpu_baseline"] = {"value": None, "unit": "tok/s", "cores": None, "kind": "port",
                                   "sample": f"failed: {ex}"}
    eng.close()
    if not a.quick:
        # the other configurations, each in its own engine after the 8B one is released
        for key, leg in (("llama_1b", lambda: llama_1b_leg(vsl, a.eager, kernel_timing=not a.no_kernel_timing)),
                         ("gemv_sweep", lambda: sweep_leg(vsl, graph=not a.eager)),
                         ("long_context", lambda: long_leg(vsl, 128, a.eager)),
                         ("llama_70b", lambda: llama_70b_leg(vsl, a.eager)),
                         ("llama_70b_q4_0", lambda: llama_70b_leg(vsl, a.eager, fmt=vsl.VSL_WF_Q4_0)),
                         ("llama_8b_q8_0", lambda: llama_8b_quant_leg(vsl, vsl.VSL_WF_Q8_0, a.eager)),
                         ("llama_8b_q4_0", lambda: llama_8b_quant_leg(vsl, vsl.VSL_WF_Q4_0, a.eager))):
            try:
                out[key] = leg()
            except Exception as ex:  # reported, never fatal to the headline measurement
                out[key] = {"failed": str(ex)}
    if a.copy_calibration_mb:
        out["copy_calibration_bytes"] = copy_calibration(vsl, a.copy_calibration_mb)
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
