"""GGUF test files: ``moe_model`` builds a small but complete qwen3moe file from the oracle's
seeded layers: every tensor the reference's qms_model_load needs (src/model.c:320-362), MoE
tensors from ``oracle.Layer`` and the rest filler, optionally split into "-0000k-of-0000n.gguf"
shards. The format itself is written by large_model_amd.gguf_writer.
"""
from __future__ import annotations

from typing import Sequence

import numpy as np

from large_model_amd.gguf_writer import (ARR, BOOL, F32, F64, I8, I16, I32, I64, STR, U8, U16, U32,  # noqa: F401
                                         U64, write_gguf, write_split)

T_F32, T_Q4_0, T_Q4_1, T_Q6_K = 0, 2, 3, 14


def moe_model(path: str, layers: Sequence, eps: float = 1e-6, n_shards: int = 1, seed: int = 99,
              n_head: int = 2, n_head_kv: int = 1, head_dim: int = 64, vocab: int = 64):
    """A qwen3moe GGUF whose layer l holds oracle.Layer ``layers[l]`` (router, gate/up/down
    experts in their own types) and a random ffn_norm; returns (path to open, norms [L][E])."""
    L0 = layers[0]
    E, X, K, F = L0.E, L0.X, L0.K, L0.F
    rng = np.random.default_rng(seed)
    f32 = lambda *shape: (rng.standard_normal(shape) * 0.02).astype(np.float32)  # noqa: E731
    kvs = [
        ("general.architecture", STR, "qwen3moe"),
        ("general.name", STR, "qmsg loader test"),
        ("general.alignment", U32, 32),
        ("qwen3moe.block_count", U32, len(layers)),
        ("qwen3moe.context_length", U32, 4096),
        ("qwen3moe.embedding_length", U32, E),
        ("qwen3moe.attention.head_count", U32, n_head),
        ("qwen3moe.attention.head_count_kv", U32, n_head_kv),
        ("qwen3moe.attention.key_length", U32, head_dim),
        ("qwen3moe.attention.value_length", U32, head_dim),
        ("qwen3moe.expert_count", U32, X),
        ("qwen3moe.expert_used_count", U32, K),
        ("qwen3moe.expert_feed_forward_length", U32, F),
        ("qwen3moe.attention.layer_norm_rms_epsilon", F32, eps),
        ("qwen3moe.rope.freq_base", F32, 5000000.0),
        ("tokenizer.ggml.tokens", ARR, (STR, [f"t{i}" for i in range(vocab)])),
        ("tokenizer.ggml.token_type", ARR, (I32, [1] * vocab)),
    ]
    tensors = [("token_embd.weight", T_F32, [E, vocab], f32(vocab, E).tobytes()),
               ("output_norm.weight", T_F32, [E], np.ones(E, np.float32).tobytes())]
    norms = []
    for l, lay in enumerate(layers):
        assert (lay.E, lay.X, lay.K, lay.F) == (E, X, K, F)
        norm = (1.0 + rng.standard_normal(E) * 0.1).astype(np.float32)
        norms.append(norm)
        b = f"blk.{l}."
        tensors += [
            (b + "attn_norm.weight", T_F32, [E], np.ones(E, np.float32).tobytes()),
            (b + "attn_q.weight", T_F32, [E, n_head * head_dim], f32(n_head * head_dim, E).tobytes()),
            (b + "attn_k.weight", T_F32, [E, n_head_kv * head_dim], f32(n_head_kv * head_dim, E).tobytes()),
            (b + "attn_v.weight", T_F32, [E, n_head_kv * head_dim], f32(n_head_kv * head_dim, E).tobytes()),
            (b + "attn_output.weight", T_F32, [n_head * head_dim, E], f32(E, n_head * head_dim).tobytes()),
            (b + "attn_q_norm.weight", T_F32, [head_dim], np.ones(head_dim, np.float32).tobytes()),
            (b + "attn_k_norm.weight", T_F32, [head_dim], np.ones(head_dim, np.float32).tobytes()),
            (b + "ffn_norm.weight", T_F32, [E], norm.tobytes()),
            (b + "ffn_gate_inp.weight", T_F32, [E, X], lay.router.tobytes()),
            (b + "ffn_gate_exps.weight", lay.types[0], [E, F, X], lay.gate.tobytes()),
            (b + "ffn_up_exps.weight", lay.types[1], [E, F, X], lay.up.tobytes()),
            (b + "ffn_down_exps.weight", lay.types[2], [F, E, X], lay.down.tobytes()),
        ]
    if n_shards == 1:
        write_gguf(path, kvs, tensors)
        return path, np.stack(norms)
    stem = path[:-5] if path.endswith(".gguf") else path
    return write_split(stem, n_shards, kvs, tensors)[0], np.stack(norms)
