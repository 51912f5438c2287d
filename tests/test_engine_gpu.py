"""End-to-end parity of the MI355X engine (VulkanSymbioteEngine token loop) against the oracle and
the committed golden vectors, through the engine C ABI."""
import os
import subprocess

import numpy as np
import pytest

import vsl_testlib

pytestmark = pytest.mark.gpu

GOLD = os.path.join(vsl_testlib.GOLDEN, "tiny_fp32.npz")
TINY = dict(hidden_size=256, num_layers=2, num_heads=4, num_kv_heads=4, intermediate_size=688, vocab_size=4096,
            max_position_embeddings=2048, rope_theta=10000.0, rms_eps=1e-5, dtype=0)


@pytest.fixture(scope="module")
def tiny_path(vsl, tmp_path_factory):
    p = tmp_path_factory.mktemp("tiny") / "tiny.gguf"
    vsl.write_synthetic_gguf(p, TINY, seed=0)
    return p


def test_tiny_fp32_golden(vsl, orc, tiny_path):
    """Tiny fp32 workload: greedy 32 tokens identical, logits within 1e-4 relative."""
    g = np.load(GOLD)
    with vsl.Engine(tiny_path, kv_capacity=64) as e:
        toks, lg = e.generate_ids(g["prompt"], 32, return_logits=True)
        assert np.array_equal(toks, g["tokens"])
        scale = np.max(np.abs(g["logits_head"]))
        assert np.max(np.abs(lg[:4] - g["logits_head"])) < 1e-4 * scale
        assert np.max(np.abs(lg.max(1) - g["logits_max"])) < 1e-4 * scale
        # eager (no hipGraph) reproduces the replayed graph bit for bit
    with vsl.Engine(tiny_path, kv_capacity=64, use_graph=False) as e2:
        t2, l2 = e2.generate_ids(g["prompt"], 32, return_logits=True)
        assert np.array_equal(t2, toks) and np.array_equal(l2, lg)


def test_tiny_stop_on_eos_capacity_and_text(vsl, orc, tiny_path):
    g = np.load(GOLD)
    m = orc.Model(tiny_path)
    with vsl.Engine(tiny_path, kv_capacity=48) as e:
        full = e.generate_ids(g["prompt"], 32)
        stop = e.generate_ids(g["prompt"], 32, stop_on_eos=True)
        assert np.array_equal(stop, m.generate(g["prompt"], 32, stop_on_eos=True))
        assert np.array_equal(stop, full[:len(stop)])
        with pytest.raises(vsl.VslError):
            e.generate_ids(g["prompt"], 34)  # 16 + 34 - 1 positions > capacity 48
        with pytest.raises(vsl.VslError):
            e.generate_ids(np.zeros(0, np.uint32), 4)
        assert len(e.generate_ids(g["prompt"], 33)) == 33  # exactly fills the cache
        # text path: prompt + one character per token (Tokenizer.cpp byte fallback)
        out = e.generate("hello world", max_tokens=5, temperature=0.0)
        assert out.startswith("hello world") and len(out) <= len("hello world") + 5
        ids = [ord(c) for c in "helloworld"]
        ref = m.generate(np.array(ids, np.uint32), 5, stop_on_eos=True)
        assert out == "hello world" + "".join(chr(t % 256) for t in ref)


def test_integration_program_runs(vsl, orc, tiny_path, tmp_path):
    """The C++ drop-in program (tests/cpp/integration_app.cpp: ConfigManager from the command line,
    VulkanSymbioteEngine(path), generate(text, 8, 0.0), run_benchmark) on the tiny model: the text
    equals the oracle's greedy continuation of the byte-fallback ids, the benchmark reports a rate."""
    from test_cpp_api import compile_cpp
    exe = compile_cpp(vsl, "integration_app.cpp", tmp_path / "integration_app")
    r = subprocess.run([exe, "--model", str(tiny_path), "hello world"], capture_output=True, timeout=300)
    assert r.returncode == 0, r.stderr.decode(errors="replace")
    m = orc.Model(tiny_path)
    ref = m.generate(np.array([ord(c) for c in "helloworld"], np.uint32), 8, stop_on_eos=True)
    m.close()
    want = b"generate: hello world" + bytes(int(t) % 256 for t in ref) + b"\n"
    assert r.stdout.startswith(want), (r.stdout[:80], want)
    bench = r.stdout[len(want):].decode().split()
    assert bench[0] == "benchmark:" and float(bench[1]) > 0 and float(bench[2]) <= float(bench[3])


def test_text_path_with_gguf_vocabulary(vsl, orc, tmp_path):
    """generate(text) with the model file's vocabulary (array and keyed layouts): the prompt encoded
    by the oracle's tokenizer, greedy ids from the oracle model (EOS 0/2 stops), and the output
    prompt + decode({id}) of each generated token, byte for byte."""
    from oracle import tokenizer as otok
    vocab = [b"<unk>", b"<s>", b"</s>"] + [bytes([i]) for i in range(32, 127)] + \
            [b"tok%d" % i for i in range(TINY["vocab_size"] - 98)]
    for keyed in (False, True):
        p = tmp_path / f"tiny_vocab_{int(keyed)}.gguf"
        vsl.write_synthetic_gguf(p, TINY, seed=0, vocab=vocab, keyed=keyed)
        tok = otok.from_gguf(p)
        m = orc.Model(p)
        with vsl.Engine(p, kv_capacity=64) as e:
            for prompt in (b"hello world", b"tok5 tok77 zz\xc3\xa9", b"   "):
                ref = m.generate(np.array(tok.encode(prompt), np.uint32), 20, stop_on_eos=True)
                want = prompt + b"".join(tok.decode([int(t)]) for t in ref)
                assert e.generate(prompt, max_tokens=20, temperature=0.0, raw=True) == want
        m.close()


def test_tiny_seeded_topk(vsl, orc, tiny_path):
    g = np.load(GOLD)
    m = orc.Model(tiny_path)
    with vsl.Engine(tiny_path, kv_capacity=64) as e:
        for seed in (1, 2):
            t = e.generate_ids(g["prompt"], 32, mode="topk", temperature=0.7, top_k=40, seed=seed)
            r = m.generate(g["prompt"], 32, sampler=orc.SAMPLE_TOPK_SEEDED, temperature=0.7, top_k=40, seed=seed)
            assert np.array_equal(t, r)
        # reference mode (T > 0 through the member top_k_sampling): the first index of the largest
        # softmax probability, which on these logits is the greedy token
        t = e.generate_ids(g["prompt"], 32, mode="reference", temperature=0.7)
        r = m.generate(g["prompt"], 32, sampler=orc.SAMPLE_REFERENCE, temperature=0.7)
        assert np.array_equal(t, r) and np.array_equal(t, g["tokens"])
        with pytest.raises(vsl.VslError):  # k = 0 is refused
            e.generate_ids(g["prompt"], 4, mode="topk", temperature=0.7, top_k=0, seed=1)
        assert len(e.generate_ids(g["prompt"], 4, mode="topk", temperature=0.7, top_k=64, seed=1)) == 4
        # top_k above V (4096) means all of V: four chunks of 1024 candidates
        t = e.generate_ids(g["prompt"], 8, mode="topk", temperature=1.0, top_k=5000, seed=4)
        r = m.generate(g["prompt"], 8, sampler=orc.SAMPLE_TOPK_SEEDED, temperature=1.0, top_k=5000, seed=4)
        assert np.array_equal(t, r)
        # k past the one-wave path (the radix select), against the oracle
        t = e.generate_ids(g["prompt"], 16, mode="topk", temperature=0.9, top_k=300, seed=3)
        r = m.generate(g["prompt"], 16, sampler=orc.SAMPLE_TOPK_SEEDED, temperature=0.9, top_k=300, seed=3)
        assert np.array_equal(t, r)


def _oracle_from_engine(orc, e, cfg):
    """Oracle model over the engine's resident weights (device -> host copies of every pack)."""
    d, L, nq, nkv, F, V = (cfg["hidden_size"], cfg["num_layers"], cfg["num_heads"], cfg["num_kv_heads"],
                           cfg["intermediate_size"], cfg["vocab_size"])
    hd = d // nq
    es = 2 if cfg["dtype"] == 1 else 4
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
        m.set_tensor(n, e.read_tensor(n, cnt * es), copy=True)
    for n in ["output_norm.weight"] + [f"blk.{l}.{s}.weight" for l in range(L) for s in ("attn_norm", "ffn_norm")]:
        m.set_tensor(n, e.read_tensor(n, d * 4), copy=True)
    assert m.check() == 0
    return m


def _forced_parity(e, m, prompt, n_new, tol, runs=None, kv_f16=True):
    """The oracle generates from the prompt (greedy unless `runs` says otherwise), then the engine is
    teacher-forced with the oracle's tokens, so both compute every step on the same token history:
    every step's logits within max-abs `tol`, and the engine's own pick at every step equal to the
    oracle's (greedy identity, or the seeded sampler's pick).  A mismatch names its step with the
    oracle's top1-top2 margin and the logit error there.  Returns the per-step oracle margins and
    logit errors of each run."""
    runs = runs or [dict(n=n_new)]
    ref = m.continuations(prompt, runs, kv_f16=kv_f16)
    report = []
    for r, (rt, rl) in zip(runs, ref):
        kw = dict(mode={0: "greedy", 1: "reference", 2: "topk"}[r.get("sampler", 0)],
                  temperature=r.get("temperature", 0.0), top_k=r.get("top_k", 40), seed=r.get("seed", 0))
        toks, lg = e.generate_ids(prompt, r["n"], return_logits=True, forced=rt[:-1], **kw)
        assert len(toks) == r["n"]
        srt = np.sort(rl, axis=1)
        margins = srt[:, -1] - srt[:, -2]
        err = np.max(np.abs(lg - rl), axis=1)
        bad = [i for i in range(r["n"]) if toks[i] != rt[i]]
        print(f"run {r}: max logit error {err.max():.5f}, smallest oracle margin {margins.min():.5f} "
              f"(step {int(np.argmin(margins))})")
        assert err.max() < tol, f"logits: step {int(np.argmax(err))} error {err.max():.5f} (tol {tol})"
        assert not bad, (f"engine pick differs from the oracle's at steps {bad}: margins "
                         f"{[round(float(margins[i]), 5) for i in bad]}, logit errors {[round(float(err[i]), 5) for i in bad]}")
        report.append((margins, err))
    return report


def test_forced_history_feeds_the_given_tokens(vsl, orc, tiny_path):
    """Teacher forcing itself: the engine forced with its own greedy tokens reproduces its free run bit
    for bit; forced with another history, its logits equal the oracle's on that history (tiny fp32
    model, 1e-4 relative)."""
    g = np.load(GOLD)
    with vsl.Engine(tiny_path, kv_capacity=64) as e:
        toks, lg = e.generate_ids(g["prompt"], 32, return_logits=True)
        t2, l2 = e.generate_ids(g["prompt"], 32, return_logits=True, forced=toks[:-1])
        assert np.array_equal(t2, toks) and np.array_equal(l2, lg)
        hist = np.random.default_rng(4).integers(0, 4096, 31).astype(np.uint32)
        t3, l3 = e.generate_ids(g["prompt"], 32, return_logits=True, forced=hist)
        with pytest.raises(vsl.VslError):
            e.generate_ids(g["prompt"], 32, forced=hist[:20])  # fewer than max_new - 1 forced ids
    m = orc.Model(tiny_path)
    ref = m.teacher_forced(np.concatenate([g["prompt"], hist]), 32)
    m.close()
    scale = np.max(np.abs(ref))
    assert np.max(np.abs(l3 - ref)) < 1e-4 * scale
    assert np.array_equal(t3, np.argmax(ref, axis=1))


def test_out_of_range_prompt_ids(vsl, orc, tiny_path):
    """Prompt ids at or past the vocabulary read embedding row V - 1 (embedding_lookup.comp:32), in the
    per-token prompt pass (tiny fp32) and in the MFMA prompt pass (1B fp16): tokens and logits equal
    the oracle's, which clamps the same way, and equal a run with the ids replaced by V - 1."""
    g = np.load(GOLD)
    prompt = g["prompt"].copy()
    prompt[[2, 9]] = [4096, 2**32 - 1]
    m = orc.Model(tiny_path)
    rt, rl = m.generate(prompt, 16, logits=True)
    m.close()
    with vsl.Engine(tiny_path, kv_capacity=64) as e:
        toks, lg = e.generate_ids(prompt, 16, return_logits=True)
        t2, l2 = e.generate_ids(np.minimum(prompt, 4095), 16, return_logits=True)
    assert np.array_equal(toks, rt) and np.array_equal(toks, t2) and np.array_equal(lg, l2)
    assert np.max(np.abs(lg - rl)) < 1e-4 * np.max(np.abs(rl))
    cfg = vsl.LLAMA_1B
    prompt = orc.random_ids(64, cfg["vocab_size"], 1)
    prompt[[0, 40]] = [cfg["vocab_size"], cfg["vocab_size"] + 12345]
    with vsl.Engine(spec=cfg, seed=0, kv_capacity=128, batched_prefill=True) as e:
        m = _oracle_from_engine(orc, e, cfg)
        _forced_parity(e, m, prompt, 8, 2e-2)
        t1, l1 = e.generate_ids(prompt, 8, return_logits=True)
        t2, l2 = e.generate_ids(np.minimum(prompt, cfg["vocab_size"] - 1), 8, return_logits=True)
    m.close()
    assert np.array_equal(t1, t2) and np.array_equal(l1, l2)


def test_windowed_mode_tiny(vsl, orc, tiny_path):
    """Windowed long-context mode with small parameters so that the run crosses the threshold
    (window 8, 4 global tokens, threshold 24; prompt 16 + 32 tokens): greedy tokens identical to the
    oracle with the same window and logits within 1e-4 relative; the steps before the threshold equal
    the dense run, the later ones differ from it."""
    g = np.load(GOLD)
    m = orc.Model(tiny_path)
    m.set_window(8, 4, 24)
    ref_toks, ref_lg = m.generate(g["prompt"], 32, logits=True)
    m.close()
    with vsl.Engine(tiny_path, kv_capacity=64, window=(8, 4, 24)) as e:
        toks, lg = e.generate_ids(g["prompt"], 32, return_logits=True)
        assert e.config["dtype"] == 0
    with vsl.Engine(tiny_path, kv_capacity=64) as e:
        dtoks, dlg = e.generate_ids(g["prompt"], 32, return_logits=True)
    scale = np.max(np.abs(ref_lg))
    assert np.array_equal(toks, ref_toks)
    assert np.max(np.abs(lg - ref_lg)) < 1e-4 * scale
    # step i samples from position 15 + i: windowed once 16 + i > 24
    assert np.max(np.abs(lg[:9] - dlg[:9])) < 1e-4 * scale
    assert np.max(np.abs(lg[9:] - dlg[9:])) > 1e-2 * scale


def test_windowed_mode_1b_batched_prefill(vsl, orc):
    """1B fp16 with the MFMA prefill crossing the threshold inside the prompt (window 16, 4 globals,
    threshold 64, prompt 128): 32 teacher-forced steps against the oracle over the resident weights
    with the same window -- logits within max-abs 2e-2 at every step, greedy picks identical."""
    cfg = vsl.LLAMA_1B
    win = (16, 4, 64)
    with vsl.Engine(spec=cfg, seed=0, kv_capacity=512, batched_prefill=True, window=win) as e:
        m = _oracle_from_engine(orc, e, cfg)
        m.set_window(*win)
        _forced_parity(e, m, orc.random_ids(128, cfg["vocab_size"], 1), 32, 2e-2)
    m.close()


@pytest.mark.parametrize("batched", [False, True])
def test_llama_1b_fp16_parity(vsl, orc, batched):
    """1B-class fp16 (GQA 32/8, head_dim 64): prompt 128, 32 teacher-forced steps against the oracle
    over the resident weights -- logits within max-abs 2e-2 at every step, greedy picks identical --
    for the per-token and the MFMA prompt pass."""
    cfg = vsl.LLAMA_1B
    with vsl.Engine(spec=cfg, seed=0, kv_capacity=512, batched_prefill=batched) as e:
        m = _oracle_from_engine(orc, e, cfg)
        _forced_parity(e, m, orc.random_ids(128, cfg["vocab_size"], 1), 32, 2e-2)
    m.close()


@pytest.mark.slow
@pytest.mark.timeout(900)
def test_llama_8b_fp16_parity(vsl, orc):
    """The 8B-class fp16 configuration as benchmarked (head_dim 128, theta 500000): the 512-token prompt
    through the MFMA prompt pass (one 512-row chunk: K-split QKV / O / down projections with their fused
    RoPE + cache append and residual + RMSNorm consumers, flash attention on hi/lo planes), then 32
    teacher-forced decode steps against the oracle over the resident weights: logits within max-abs 2e-2
    at every step and greedy picks identical at every step."""
    cfg = vsl.LLAMA_8B
    with vsl.Engine(spec=cfg, seed=0, kv_capacity=1024, batched_prefill=True) as e:
        m = _oracle_from_engine(orc, e, cfg)
        _forced_parity(e, m, orc.random_ids(512, cfg["vocab_size"], 1), 32, 2e-2)
    m.close()


@pytest.mark.slow
@pytest.mark.timeout(900)
@pytest.mark.parametrize("fmt", ["q4_0", "q8_0"])
def test_llama_8b_resident_blocks_parity(vsl, orc, fmt):
    """The 8B-class model with every linear weight quantized on the device (Q4_0 / Q8_0) and decoded
    from the resident blocks at the full shapes (the 16-wave down projection, the 8-wave SwiGLU GEMV,
    the quantized lm_head): the expanded packs in fp32 hold exactly the blocks' values, so the oracle
    over them is the same model. A 256-token prompt (per-token steps over the blocks: an fp32 model
    has no MFMA prompt pass), then 32 teacher-forced greedy steps: logits within max-abs 2e-2 at every
    step, picks identical."""
    cfg = dict(vsl.LLAMA_8B, dtype={"q4_0": vsl.VSL_WF_Q4_0, "q8_0": vsl.VSL_WF_Q8_0}[fmt])
    with vsl.Engine(spec=cfg, seed=0, kv_capacity=512, dequant_f32=True) as e:
        assert e.config["dtype"] == 0
        m = _oracle_from_engine(orc, e, dict(cfg, dtype=0))
        _forced_parity(e, m, orc.random_ids(256, cfg["vocab_size"], 3), 32, 2e-2, kv_f16=False)
    m.close()


@pytest.mark.slow
@pytest.mark.timeout(900)
@pytest.mark.parametrize("fmt,conv", [("q4_0", "ggml"), ("q8_0", "reference")])
def test_llama_1b_quantized_file_default_path(vsl, orc, tmp_path, fmt, conv):
    """A 1B-class GGUF file with every 2-D weight block-quantized, opened with the engine's defaults:
    the blocks expanded into fp16 packs for the MFMA prompt pass (128 rows: K-split direct-to-LDS
    tiles) and kept resident for the decode GEMVs. Against the oracle that dequantizes the same file
    (fp32 weights, fp16 KV cache): 32 teacher-forced greedy steps after a 128-token prompt, logits
    within max-abs 2e-2 at every step, picks identical."""
    cfg = dict(vsl.LLAMA_1B, dtype={"q4_0": vsl.VSL_WF_Q4_0, "q8_0": vsl.VSL_WF_Q8_0}[fmt])
    p = tmp_path / f"llama1b_{fmt}.gguf"
    vsl.write_synthetic_gguf(p, cfg, seed=11, convention=conv)
    m = orc.Model(p)
    try:
        with vsl.Engine(p, kv_capacity=512) as e:
            _forced_parity(e, m, orc.random_ids(128, cfg["vocab_size"], 5), 32, 2e-2)
    finally:
        m.close()
        p.unlink()


@pytest.mark.slow
@pytest.mark.timeout(900)
def test_llama_8b_long_path_oracle(vsl, orc):
    """The full 32-layer 8B model on the long-context path against the oracle: a KV capacity of 16384
    (above 8192, so decode attention runs on the matrix-core kernel), a 768-token prompt in three
    256-row MFMA chunks (each chunk attending to the cache the previous ones filled), then 16 teacher-
    forced greedy steps and 16 teacher-forced T = 0.7 top-k 40 seeded steps on another prompt than
    the 512-token test: logits within max-abs 2e-2 at every step, picks identical."""
    cfg = vsl.LLAMA_8B
    prompt = orc.random_ids(768, cfg["vocab_size"], 7)
    with vsl.Engine(spec=cfg, seed=0, kv_capacity=16384, batched_prefill=True, prefill_chunk=256) as e:
        m = _oracle_from_engine(orc, e, cfg)
        _forced_parity(e, m, prompt, 16, 2e-2,
                       runs=[dict(n=16), dict(n=16, sampler=orc.SAMPLE_TOPK_SEEDED, temperature=0.7, top_k=40, seed=5)])
    m.close()


# A small model with the 8B attention geometry (head_dim 128, GQA 4, theta 500000) so that the oracle can
# follow an 8192-token prompt: the chunked MFMA prompt pass (four 2048-row chunks), RoPE at positions
# past 8K, and the matrix-core decode attention that caches above 8192 positions select.
LONG_SMALL = dict(hidden_size=1024, num_layers=2, num_heads=8, num_kv_heads=2, intermediate_size=2816,
                  vocab_size=32000, max_position_embeddings=32768, rope_theta=500000.0, rms_eps=1e-5, dtype=1)


@pytest.mark.slow
@pytest.mark.timeout(900)
def test_long_context_oracle_small_model(vsl, orc):
    """Long-context path against the oracle: 8192 prompt tokens in 2048-row chunks into a 32768-position
    fp16 cache, then 32 teacher-forced greedy steps (logits within max-abs 2e-2, picks identical) and 32
    teacher-forced T = 0.7 seeded top-k 40 steps (the engine's pick at every step equal to the oracle's
    Utils.cpp:140-172 restatement with the same Philox uniform)."""
    cfg = LONG_SMALL
    prompt = np.random.default_rng(11).integers(0, cfg["vocab_size"], 8192).astype(np.uint32)
    with vsl.Engine(spec=cfg, seed=0, kv_capacity=32768, batched_prefill=True, prefill_chunk=2048) as e:
        m = _oracle_from_engine(orc, e, cfg)
        _forced_parity(e, m, prompt, 32, 2e-2,
                       runs=[dict(n=32), dict(n=32, sampler=orc.SAMPLE_TOPK_SEEDED, temperature=0.7, top_k=40, seed=7)])
    m.close()


# Model dimensions that are odd multiples of 128 (d 640, [Wq; Wk; Wv] 1920 rows), with an FFN wide enough
# that a prompt chunk of 128 rows or more takes the 64 x 128 direct-to-LDS tiles for gate/up at K = 640
# (ten 64-column stages: four-stage rounds and a closing pair); the narrow projections run on the
# register-staged tiles.
ODD128 = dict(hidden_size=640, num_layers=2, num_heads=5, num_kv_heads=5, intermediate_size=6144,
              vocab_size=32000, max_position_embeddings=4096, rope_theta=10000.0, rms_eps=1e-5, dtype=1)


@pytest.mark.parametrize("chunk", [128, 299, 0])
def test_odd_multiple_of_128_dimensions(vsl, orc, chunk):
    """d = 640 (head_dim 128, five heads, no GQA) against the oracle: a 300-token prompt through the
    MFMA prompt pass in 128-row chunks (128, 128, 44 rows), in chunks of 299 and 1 rows, or in one
    300-row chunk, then 24 teacher-forced greedy steps: logits within max-abs 2e-2 at every step, picks
    identical."""
    cfg = ODD128
    with vsl.Engine(spec=cfg, seed=0, kv_capacity=512, batched_prefill=True, prefill_chunk=chunk) as e:
        m = _oracle_from_engine(orc, e, cfg)
        _forced_parity(e, m, orc.random_ids(300, cfg["vocab_size"], 3), 24, 2e-2)
    m.close()


# Three query heads per KV head (the Llama-3.2-3B grouping, 24 / 8 heads), at head_dim 128.
GQA3 = dict(hidden_size=768, num_layers=2, num_heads=6, num_kv_heads=2, intermediate_size=2048,
            vocab_size=32000, max_position_embeddings=4096, rope_theta=500000.0, rms_eps=1e-5, dtype=1)


@pytest.mark.parametrize("batched,cap", [(True, 1024), (False, 1024), (True, 9216)])
def test_gqa_group_of_three(vsl, orc, batched, cap):
    """GQA with three query heads per KV head against the oracle: a 200-token prompt through the MFMA
    prompt pass (one head per attention block) or the per-token pass, then 24 teacher-forced greedy
    steps on the vector decode attention (capacity 1024) or the matrix-core one (capacity 9216):
    logits within max-abs 2e-2 at every step, picks identical."""
    cfg = GQA3
    with vsl.Engine(spec=cfg, seed=0, kv_capacity=cap, batched_prefill=batched) as e:
        m = _oracle_from_engine(orc, e, cfg)
        _forced_parity(e, m, orc.random_ids(200, cfg["vocab_size"], 5), 24, 2e-2)
    m.close()


# Eight query heads per KV head (the 70B-class grouping, 64 / 8 heads) at head_dim 128 and 64.
GQA8 = {128: dict(hidden_size=2048, num_layers=2, num_heads=16, num_kv_heads=2, intermediate_size=4096,
                  vocab_size=32000, max_position_embeddings=4096, rope_theta=500000.0, rms_eps=1e-5, dtype=1),
        64: dict(hidden_size=1024, num_layers=2, num_heads=16, num_kv_heads=2, intermediate_size=2816,
                 vocab_size=32000, max_position_embeddings=4096, rope_theta=10000.0, rms_eps=1e-5, dtype=1)}


@pytest.mark.parametrize("hd,batched,cap", [(128, True, 1024), (128, False, 1024), (128, True, 9216),
                                            (64, True, 1024), (64, False, 1024)])
def test_gqa_group_of_eight(vsl, orc, hd, batched, cap):
    """GQA with eight query heads per KV head against the oracle: a 200-token prompt through the MFMA
    prompt pass or the per-token pass, then 24 teacher-forced greedy steps on the vector decode
    attention (capacity 1024) or, at head_dim 128, the matrix-core one (capacity 9216): logits within
    max-abs 2e-2 at every step, picks identical."""
    cfg = GQA8[hd]
    with vsl.Engine(spec=cfg, seed=0, kv_capacity=cap, batched_prefill=batched) as e:
        m = _oracle_from_engine(orc, e, cfg)
        _forced_parity(e, m, orc.random_ids(200, cfg["vocab_size"], 6), 24, 2e-2)
    m.close()


# An FFN wider than 16384 (the 70B-class 28672 needs the same path): the decode down projection stages
# its 20480-wide input with one 16-wave block per CU.
WIDE_FFN = dict(hidden_size=512, num_layers=2, num_heads=4, num_kv_heads=1, intermediate_size=20480,
                vocab_size=4096, max_position_embeddings=4096, rope_theta=10000.0, rms_eps=1e-5, dtype=1)


def test_ffn_wider_than_16384(vsl, orc):
    """FFN 20480 against the oracle: a 256-token prompt through the MFMA prompt pass, then 24 teacher-
    forced greedy steps: logits within max-abs 2e-2 at every step, picks identical."""
    cfg = WIDE_FFN
    with vsl.Engine(spec=cfg, seed=0, kv_capacity=512, batched_prefill=True) as e:
        m = _oracle_from_engine(orc, e, cfg)
        _forced_parity(e, m, orc.random_ids(256, cfg["vocab_size"], 9), 24, 2e-2)
    m.close()


def _plant_outliers(vsl, path, names, values, per_tensor, seed):
    """Overwrite `per_tensor` random fp16 weights of each named tensor of a GGUF file in place with
    `values` (cycled); the file's other bytes are unchanged."""
    import ctypes
    L = vsl.engine_lib()
    h = ctypes.c_void_p()
    vsl.check(L.vsl_gguf_open(str(path).encode(), ctypes.byref(h)), L)
    rng = np.random.default_rng(seed)
    try:
        mm = np.memmap(path, dtype=np.uint8, mode="r+")
        for n in names:
            off, size, rt, nd = ctypes.c_uint64(), ctypes.c_uint64(), ctypes.c_uint32(), ctypes.c_uint32()
            dims = (ctypes.c_uint64 * 4)()
            vsl.check(L.vsl_gguf_tensor(h, n.encode(), ctypes.byref(off), ctypes.byref(size), ctypes.byref(rt),
                                        ctypes.byref(nd), dims), L)
            w = mm[off.value:off.value + size.value].view(np.float16)
            idx = rng.choice(w.size, per_tensor, replace=False)
            w[idx] = np.resize(np.asarray(values, np.float16), per_tensor)
        mm.flush()
        del mm
    finally:
        L.vsl_gguf_close(h)


@pytest.mark.slow
@pytest.mark.timeout(900)
def test_fp8_prefill_with_outlier_weights(vsl, orc, tmp_path):
    """The prompt pass's fp8 lo products on a model file whose gate/up, down and O weights hold outliers
    (+-7.5 and +-40 among N(0, 0.02): past e4m3's 448 at the fixed 2^6 weight scale). d 1024 and FFN 2816
    with a 2048-row chunk put the O, gate/up and down GEMMs on the F16F8 path; each layer's weight shift
    comes from its own largest weight. 16 teacher-forced greedy steps against the oracle reading the same
    file: every logit finite and within max-abs 2e-2, picks identical."""
    cfg = dict(LONG_SMALL, max_position_embeddings=4096)
    p = tmp_path / "outliers.gguf"
    vsl.write_synthetic_gguf(p, cfg, seed=0)
    names = [f"blk.{l}.{t}.weight" for l in range(cfg["num_layers"])
             for t in ("ffn_gate", "ffn_up", "ffn_down", "attn_o")]
    _plant_outliers(vsl, p, names, [7.5, -7.5, 40.0, -40.0], 48, 3)
    prompt = np.random.default_rng(12).integers(0, cfg["vocab_size"], 2048).astype(np.uint32)
    m = orc.Model(p)
    with vsl.Engine(p, kv_capacity=2048 + 32, batched_prefill=True, prefill_chunk=2048) as e:
        w = e.read_tensor("blk.1.ffn_down.weight", 2 * cfg["hidden_size"] * cfg["intermediate_size"])
        assert w.dtype == np.float16 and np.max(np.abs(w.astype(np.float32))) == 40.0
        rep = _forced_parity(e, m, prompt, 16, 2e-2)
        toks, lg = e.generate_ids(prompt, 4, return_logits=True)
        assert np.all(np.isfinite(lg))
    m.close()
    assert rep and np.all(np.isfinite(rep[0][1]))


def test_engine_stats_and_packs(vsl):
    with vsl.Engine(spec=vsl.LLAMA_1B, kv_capacity=512) as e:
        cfg = e.config
        assert cfg["head_dim"] == 64 and cfg["dtype"] == 1
        wb = e.weight_bytes()
        # 2 * (L * (d*(nq+2nkv)*hd + nq*hd*d + 3*F*d) + 2*V*d) + fp32 norm gains
        d, L, F, V = 2048, 16, 8192, 32000
        lin = L * (d * (32 + 16) * 64 + 32 * 64 * d + 3 * F * d) + 2 * V * d
        assert wb == 2 * lin + 4 * d * (2 * L + 1)
        assert e.kv_bytes() == 2 * L * 8 * 512 * 64 * 2
        st = e.vram_stats()
        assert st["used_size"] >= wb + e.kv_bytes() and st["total_size"] >= st["used_size"]
        e.generate_ids(np.arange(1, 17, dtype=np.uint32), 8)
        s = e.last_stats()
        assert s["prompt_tokens"] == 16 and s["generated_tokens"] == 8 and s["decode_ms"] > 0
        # one resident pack per tensor, each in HBM (tier VRAM_HOT) inside the arena, sized as stored
        packs = e.packs()
        assert len(packs) == 9 * L + 3
        assert sum(p["resident_bytes"] for p in packs) == wb
        assert all(p["tier"] == 0 and p["device_ptr"] for p in packs)
        by = {p["name"]: p for p in packs}
        assert by["blk.3.ffn_down.weight"]["resident_bytes"] == 2 * d * F and by["blk.3.ffn_down.weight"]["dtype"] == 1
        assert by["blk.3.ffn_norm.weight"]["dtype"] == 0 and by["blk.3.ffn_norm.weight"]["resident_bytes"] == 4 * d
        assert (by["blk.3.attn_q.weight"]["type"], by["blk.3.attn_q.weight"]["layer_idx"]) == (0, 3)
        assert by["blk.3.ffn_up.weight"]["type"] == 4 and by["output_norm.weight"]["type"] == 11
        # the q/k/v packs of a layer are contiguous (one fused GEMV reads them as one matrix)
        q, k, v = (by[f"blk.7.attn_{x}.weight"] for x in "qkv")
        assert k["device_ptr"] == q["device_ptr"] + q["resident_bytes"]
        assert v["device_ptr"] == k["device_ptr"] + k["resident_bytes"]
        st = e.vram_stats()
        assert st["used_size"] >= wb


@pytest.mark.slow
@pytest.mark.timeout(900)
def test_llama_8b_long_context(vsl):
    """Long-context 8B workload at full size (too large for the oracle): an 8192-token prompt in 2048-row
    MFMA chunks into a 32768-position fp16 KV cache against the per-token path (the decode kernels the
    oracle pins) on the same weights, teacher-forced with the per-token path's greedy tokens: logits
    within max-abs 2e-2 and picks identical at all 8 steps; seeded T = 0.7 sampling reproducible per
    seed, seed-dependent and in range."""
    cfg = vsl.LLAMA_8B
    V = cfg["vocab_size"]
    prompt = np.random.default_rng(11).integers(0, V, 8192).astype(np.uint32)
    n_new = 8
    with vsl.Engine(spec=cfg, seed=0, kv_capacity=32768, batched_prefill=False) as e:
        rt, rl = e.generate_ids(prompt, n_new, return_logits=True)
    with vsl.Engine(spec=cfg, seed=0, kv_capacity=32768, batched_prefill=True) as e:
        toks, lg = e.generate_ids(prompt, n_new, return_logits=True, forced=rt[:-1])
        s1 = e.generate_ids(prompt, 32, mode="topk", temperature=0.7, top_k=40, seed=7)
        s2 = e.generate_ids(prompt, 32, mode="topk", temperature=0.7, top_k=40, seed=7)
        s3 = e.generate_ids(prompt, 32, mode="topk", temperature=0.7, top_k=40, seed=8)
    srt = np.sort(rl, axis=1)
    margins = srt[:, -1] - srt[:, -2]
    err = np.max(np.abs(lg - rl), axis=1)
    print(f"max logit error {err.max():.5f}, smallest reference margin {margins.min():.5f}")
    assert err.max() < 2e-2, err
    bad = [i for i in range(n_new) if toks[i] != rt[i]]
    assert not bad, f"picks differ at {bad}: margins {margins[bad]}, errors {err[bad]}"
    assert np.array_equal(s1, s2) and not np.array_equal(s1, s3)
    assert len(s1) == 32 and int(s1.max()) < V and int(s3.max()) < V
