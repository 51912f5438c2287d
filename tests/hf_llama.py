"""Independent textbook check: a transformers LlamaForCausalLM built from a local config (nothing is
downloaded) with the weights of a GGUF file.

transformers rotates (j, j + hd/2) pairs; the reference rotates adjacent pairs (2j, 2j+1)
(fused_matmul_rope.comp:48-81).  Permuting the rows of Wq and Wk inside each head by
[0, 2, 4, ..., 1, 3, 5, ...] maps one convention onto the other; scores q.k are unchanged because
q and k are permuted alike.
"""
import numpy as np


def read_gguf_tensors(orc, path, names):
    import ctypes
    L = orc.lib()
    h = ctypes.c_void_p()
    assert L.orc_gguf_open(str(path).encode(), ctypes.byref(h)) == 0
    out = {}
    try:
        for n in names:
            idx = L.orc_gguf_find(h, n.encode())
            assert idx >= 0, n
            nd = ctypes.c_uint32()
            dims = (ctypes.c_uint64 * 4)()
            L.orc_gguf_tensor_info(h, idx, None, 0, ctypes.byref(nd), dims, None, None, None)
            shape = [dims[i] for i in range(nd.value)][::-1]
            buf = np.zeros(int(np.prod(shape)), np.float32)
            assert L.orc_gguf_read_f32(h, n.encode(), orc.ptr(buf), buf.size) == buf.size
            out[n] = buf.reshape(shape)
    finally:
        L.orc_gguf_close(h)
    return out


def build(orc, path, cfg):
    import torch
    from transformers import LlamaConfig, LlamaForCausalLM
    d, L, nq, nkv = cfg["hidden_size"], cfg["num_layers"], cfg["num_heads"], cfg["num_kv_heads"]
    hd = d // nq
    hc = LlamaConfig(vocab_size=cfg["vocab_size"], hidden_size=d, intermediate_size=cfg["intermediate_size"],
                     num_hidden_layers=L, num_attention_heads=nq, num_key_value_heads=nkv,
                     rms_norm_eps=cfg["rms_eps"], rope_theta=cfg["rope_theta"],
                     max_position_embeddings=cfg.get("max_position_embeddings", 2048), tie_word_embeddings=False,
                     attention_bias=False, mlp_bias=False, attn_implementation="eager")
    model = LlamaForCausalLM(hc).float().eval()
    names = ["token_embd.weight", "output_norm.weight", "output.weight"]
    for l in range(L):
        names += [f"blk.{l}.{s}.weight" for s in ("attn_norm", "attn_q", "attn_k", "attn_v", "attn_o", "ffn_norm",
                                                   "ffn_gate", "ffn_up", "ffn_down")]
    w = read_gguf_tensors(orc, path, names)
    perm = np.concatenate([np.arange(0, hd, 2), np.arange(1, hd, 2)])

    def heads_perm(W, n):
        return W.reshape(n, hd, -1)[:, perm, :].reshape(n * hd, -1)

    sd = {"model.embed_tokens.weight": w["token_embd.weight"], "model.norm.weight": w["output_norm.weight"],
          "lm_head.weight": w["output.weight"]}
    for l in range(L):
        p = f"model.layers.{l}."
        sd[p + "input_layernorm.weight"] = w[f"blk.{l}.attn_norm.weight"]
        sd[p + "post_attention_layernorm.weight"] = w[f"blk.{l}.ffn_norm.weight"]
        sd[p + "self_attn.q_proj.weight"] = heads_perm(w[f"blk.{l}.attn_q.weight"], nq)
        sd[p + "self_attn.k_proj.weight"] = heads_perm(w[f"blk.{l}.attn_k.weight"], nkv)
        sd[p + "self_attn.v_proj.weight"] = w[f"blk.{l}.attn_v.weight"]
        sd[p + "self_attn.o_proj.weight"] = w[f"blk.{l}.attn_o.weight"]
        sd[p + "mlp.gate_proj.weight"] = w[f"blk.{l}.ffn_gate.weight"]
        sd[p + "mlp.up_proj.weight"] = w[f"blk.{l}.ffn_up.weight"]
        sd[p + "mlp.down_proj.weight"] = w[f"blk.{l}.ffn_down.weight"]
    model.load_state_dict({k: torch.from_numpy(np.ascontiguousarray(v)) for k, v in sd.items()}, strict=True)
    return model


def logits(model, ids):
    import torch
    with torch.no_grad():
        return model(torch.tensor([list(map(int, ids))])).logits[0].numpy()


def greedy(model, prompt, n):
    """Greedy token loop with full recomputation (no cache): argmax picks the first index of the max."""
    import torch
    ids = list(map(int, prompt))
    out = []
    with torch.no_grad():
        for _ in range(n):
            lg = model(torch.tensor([ids])).logits[0, -1]
            t = int(torch.argmax(lg))
            out.append(t)
            ids.append(t)
    return np.array(out, np.uint32)
