"""A tiny Llama-architecture GGUF model for the prompt-forward tests.

Test infrastructure: the file is fully determined by `seed` (block streams
from holo_mi355x.synth, norm weights from numpy's default_rng), so the GPU box
rebuilds the same bytes the golden fixture was computed on.  Shapes: 2 layers,
dim 256, 8 query heads and 4 KV heads of 32 (grouped-query attention), FFN
512, vocabulary 320, context 256.  Types mix the hot formats: Q4_0 embedding
and projections, Q8_0 value projection and output head, and a down projection
whose type differs per layer (Q4_K, then Q6_K), as in mixed-quant files.
"""
from __future__ import annotations

import numpy as np

import gguf_files as gf

CFG = dict(n_layers=2, dim=256, n_heads=8, n_kv_heads=4, head_dim=32, ffn=512, vocab=320, ctx=256)
KV_DIM = CFG["n_kv_heads"] * CFG["head_dim"]
DOWN_TYPES = (12, 14)


def build(path, seed: int = 7) -> None:
    from holo_mi355x import synth
    c = CFG
    rng = np.random.default_rng(seed)
    kvs = [("general.architecture", gf.STR, "llama"), ("llama.embedding_length", gf.U32, c["dim"]),
           ("llama.block_count", gf.U32, c["n_layers"]), ("llama.attention.head_count", gf.U32, c["n_heads"]),
           ("llama.attention.head_count_kv", gf.U32, c["n_kv_heads"]),
           ("llama.feed_forward_length", gf.U32, c["ffn"]), ("llama.context_length", gf.U32, c["ctx"]),
           ("llama.rope.freq_base", gf.F32, 10000.0), ("llama.attention.layer_norm_rms_epsilon", gf.F32, 1e-5),
           ("tokenizer.ggml.tokens", gf.ARR, (gf.STR, [f"t{i}" for i in range(c["vocab"])]))]
    s = [seed * 1000]

    def blocks(t, rows, cols):
        s[0] += 1
        return synth.blocks(t, rows, cols, seed=s[0]).tobytes()

    def norm(n):
        return (1.0 + 0.1 * rng.standard_normal(n)).astype(np.float32).tobytes()

    d, f, kv = c["dim"], c["ffn"], KV_DIM
    ts = [gf.Tensor("token_embd.weight", [d, c["vocab"]], 2, blocks(2, c["vocab"], d)),
          gf.Tensor("output_norm.weight", [d], 0, norm(d)),
          gf.Tensor("output.weight", [d, c["vocab"]], 8, blocks(8, c["vocab"], d))]
    for l in range(c["n_layers"]):
        b = f"blk.{l}."
        ts += [gf.Tensor(b + "attn_norm.weight", [d], 0, norm(d)),
               gf.Tensor(b + "attn_q.weight", [d, d], 2, blocks(2, d, d)),
               gf.Tensor(b + "attn_k.weight", [d, kv], 2, blocks(2, kv, d)),
               gf.Tensor(b + "attn_v.weight", [d, kv], 8, blocks(8, kv, d)),
               gf.Tensor(b + "attn_output.weight", [d, d], 2, blocks(2, d, d)),
               gf.Tensor(b + "ffn_norm.weight", [d], 0, norm(d)),
               gf.Tensor(b + "ffn_gate.weight", [d, f], 2, blocks(2, f, d)),
               gf.Tensor(b + "ffn_up.weight", [d, f], 2, blocks(2, f, d)),
               gf.Tensor(b + "ffn_down.weight", [f, d], DOWN_TYPES[l], blocks(DOWN_TYPES[l], d, f))]
    gf.write(path, kvs, ts)


def prompt(n: int, seed: int = 11) -> np.ndarray:
    return np.random.default_rng(seed).integers(0, CFG["vocab"], size=n).astype(np.int32)
