"""End-to-end pins of the oracle's token loop (VulkanSymbioteEngine::generate semantics,
VulkanSymbioteEngine.cpp:678-765) against the committed golden vectors and an independent
transformers Llama."""
import hashlib
import os

import numpy as np
import pytest

import hf_llama
import vsl_testlib

GOLD = os.path.join(vsl_testlib.GOLDEN, "tiny_fp32.npz")
TINY = dict(hidden_size=256, num_layers=2, num_heads=4, num_kv_heads=4, intermediate_size=688, vocab_size=4096,
            max_position_embeddings=2048, rope_theta=10000.0, rms_eps=1e-5)


@pytest.fixture(scope="module")
def tiny_gguf(vsl, tmp_path_factory):
    p = tmp_path_factory.mktemp("tiny") / "tiny.gguf"
    vsl.write_synthetic_gguf(p, dict(TINY, dtype=vsl.VSL_DT_F32), seed=0)
    return p


def test_golden_tiny_oracle(orc, tiny_gguf):
    g = np.load(GOLD)
    assert hashlib.sha256(tiny_gguf.read_bytes()).hexdigest() == str(g["gguf_sha256"])
    prompt = orc.random_ids(16, 4096, 1)
    assert np.array_equal(prompt, g["prompt"])
    m = orc.Model(tiny_gguf)
    toks, lg = m.generate(prompt, 32, logits=True)
    assert np.array_equal(toks, g["tokens"])
    assert np.max(np.abs(lg[:4] - g["logits_head"])) < 1e-4
    assert np.max(np.abs(lg.max(1) - g["logits_max"])) < 1e-4


def test_oracle_gqa_fp16_vs_transformers(vsl, orc, tmp_path):
    cfg = dict(hidden_size=512, num_layers=2, num_heads=8, num_kv_heads=2, intermediate_size=1024, vocab_size=1000,
               max_position_embeddings=512, rope_theta=500000.0, rms_eps=1e-5)
    p = tmp_path / "gqa.gguf"
    vsl.write_synthetic_gguf(p, dict(cfg, dtype=vsl.VSL_DT_F16), seed=7)
    model = hf_llama.build(orc, p, cfg)
    ids = orc.random_ids(24, cfg["vocab_size"], 3)
    ref = hf_llama.logits(model, ids)
    ours = orc.Model(p).teacher_forced(ids, 24)
    assert np.max(np.abs(ours - ref)) < 1e-4


def test_oracle_stop_on_eos_and_capacity(orc, tiny_gguf):
    m = orc.Model(tiny_gguf)
    prompt = orc.random_ids(16, 4096, 1)
    full = m.generate(prompt, 12)
    # forcing EOS: a prompt whose greedy continuation is known; stop_on_eos stops right after 0/2
    toks = m.generate(prompt, 12, stop_on_eos=True)
    assert np.array_equal(toks, full[:len(toks)])
    eos = [i for i, t in enumerate(full) if t in (0, 2)]
    assert len(toks) == (eos[0] + 1 if eos else 12)
    with pytest.raises(RuntimeError):
        m.generate(np.zeros(0, np.uint32), 4)


def test_oracle_token_id_clamp(orc, tiny_gguf):
    """embedding_lookup.comp:32 clamps ids to vocab-1: id 10**6 behaves as 4095."""
    m = orc.Model(tiny_gguf)
    a = m.teacher_forced(np.array([5, 4095], np.uint32), 1)
    b = m.teacher_forced(np.array([5, 10**6], np.uint32), 1)
    assert np.array_equal(a, b)


def test_oracle_continuations_match_generate(orc, tiny_gguf):
    """continuations() (one processed prompt, several runs restarting at its end) gives each run exactly
    what generate() gives from scratch: greedy and seeded top-k, tokens and logits, in either order."""
    m = orc.Model(tiny_gguf)
    prompt = orc.random_ids(16, 4096, 1)
    runs = [dict(n=12, sampler=orc.SAMPLE_TOPK_SEEDED, temperature=0.7, top_k=40, seed=3), dict(n=9)]
    got = m.continuations(prompt, runs)
    t0, l0 = m.generate(prompt, 12, sampler=orc.SAMPLE_TOPK_SEEDED, temperature=0.7, top_k=40, seed=3, logits=True)
    t1, l1 = m.generate(prompt, 9, logits=True)
    assert np.array_equal(got[0][0], t0) and np.array_equal(got[0][1], l0)
    assert np.array_equal(got[1][0], t1) and np.array_equal(got[1][1], l1)
    assert np.array_equal(t1, np.load(GOLD)["tokens"][:9])
