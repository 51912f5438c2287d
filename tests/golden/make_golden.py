"""Writes tests/golden/tiny_fp32.npz: the tiny fp32 workload's golden vectors.

Workload: Llama-style decoder, fp32, 2 layers, d_model 256, 4 heads (head_dim 64, no GQA), SwiGLU
FFN 688, vocab 4096, RMSNorm eps 1e-5, RoPE theta 10000, untied lm_head, weights N(0, 0.02) from
seed 0, norm gains 1.0, written as a GGUF file; prompt = 16 uniform-random ids (seed 1); greedy
decode 32 tokens.

The token ids and logits come from an independent transformers LlamaForCausalLM built from a local
config with the GGUF's weights (tests/hf_llama.py), not from the oracle; the script asserts that
the oracle agrees before writing.  The GGUF bytes are pinned by their SHA-256.

Run from the repository root:  python tests/golden/make_golden.py
"""
import hashlib
import os
import sys
import tempfile

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(HERE))
import vsl_testlib  # noqa: E402
import hf_llama  # noqa: E402

TINY = dict(hidden_size=256, num_layers=2, num_heads=4, num_kv_heads=4, intermediate_size=688, vocab_size=4096,
            max_position_embeddings=2048, rope_theta=10000.0, rms_eps=1e-5)
N_PROMPT, N_NEW = 16, 32


def main():
    vsl = vsl_testlib.package()
    orc = vsl_testlib.oracle()
    with tempfile.TemporaryDirectory() as td:
        path = os.path.join(td, "tiny.gguf")
        vsl.write_synthetic_gguf(path, dict(TINY, dtype=vsl.VSL_DT_F32), seed=0)
        sha = hashlib.sha256(open(path, "rb").read()).hexdigest()
        prompt = orc.random_ids(N_PROMPT, TINY["vocab_size"], 1)
        model = hf_llama.build(orc, path, TINY)
        toks = hf_llama.greedy(model, prompt, N_NEW)
        full = np.concatenate([prompt, toks[:-1]])
        lg = hf_llama.logits(model, full)[N_PROMPT - 1:]  # logits each generated token was sampled from
        om = orc.Model(path)
        otoks, olg = om.generate(prompt, N_NEW, logits=True)
        assert np.array_equal(otoks, toks), (otoks, toks)
        assert np.max(np.abs(olg - lg)) < 1e-4
        top2 = np.sort(lg, axis=1)[:, -2:]
        np.savez_compressed(os.path.join(HERE, "tiny_fp32.npz"), prompt=prompt, tokens=toks,
                            logits_head=lg[:4].astype(np.float32), logits_max=lg.max(1).astype(np.float32),
                            margin=(top2[:, 1] - top2[:, 0]).astype(np.float32), gguf_sha256=np.array(sha))
        print("tokens", toks.tolist())
        print("min top1-top2 margin", float((top2[:, 1] - top2[:, 0]).min()))


if __name__ == "__main__":
    main()
