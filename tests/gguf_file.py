"""Writing GGUF v3 files for the loader tests (test helper, no reference code).

The layout follows the published GGUF v3 format: magic "GGUF", u32 version, u64 tensor count,
u64 metadata count, metadata (string key, u32 value type, value), tensor infos (string name,
u32 n_dims, u64 ne[n_dims], u32 type, u64 offset relative to the data section), padding to
``general.alignment`` (32 unless given), then the tensor data, each tensor at an aligned
offset. Little-endian throughout.

``moe_model`` builds a small but complete qwen3moe file from the oracle's seeded layers: every
tensor the reference's qms_model_load needs (src/model.c:320-362), MoE tensors from
``oracle.Layer`` and the rest filler, optionally split into "-0000k-of-0000n.gguf" shards.
"""
from __future__ import annotations

import struct
from typing import Optional, Sequence

import numpy as np

U8, I8, U16, I16, U32, I32, F32, BOOL, STR, ARR, U64, I64, F64 = range(13)
_FMT = {U8: "<B", I8: "<b", U16: "<H", I16: "<h", U32: "<I", I32: "<i", F32: "<f", BOOL: "<B",
        U64: "<Q", I64: "<q", F64: "<d"}

T_F32, T_Q4_0, T_Q4_1, T_Q6_K = 0, 2, 3, 14


def _s(text: str) -> bytes:
    b = text.encode()
    return struct.pack("<Q", len(b)) + b


def _value(vt: int, v) -> bytes:
    if vt == STR:
        return _s(v)
    if vt == ARR:
        et, items = v
        return struct.pack("<IQ", et, len(items)) + b"".join(_value(et, x) for x in items)
    return struct.pack(_FMT[vt], v)


def _align(n: int, a: int) -> int:
    return (n + a - 1) // a * a


def write_gguf(path: str, kvs: Sequence[tuple], tensors: Sequence[tuple], alignment: int = 32,
               version: int = 3, truncate: Optional[int] = None) -> dict:
    """kvs: (key, value type, value); tensors: (name, ggml type, ne list, bytes).
    Returns {name: absolute data offset}. ``truncate`` cuts the file to that many bytes.
    An alignment other than 32 is recorded as general.alignment unless kvs already has it."""
    kvs = list(kvs)
    if alignment != 32 and not any(k[0] == "general.alignment" for k in kvs):
        kvs.append(("general.alignment", U32, alignment))
    head = b"GGUF" + struct.pack("<IQQ", version, len(tensors), len(kvs))
    for key, vt, v in kvs:
        head += _s(key) + struct.pack("<I", vt) + _value(vt, v)
    rel, off = [], 0
    for _, _, _, data in tensors:
        off = _align(off, alignment)
        rel.append(off)
        off += len(data)
    for (name, t, ne, _), o in zip(tensors, rel):
        head += _s(name) + struct.pack("<I", len(ne)) + b"".join(struct.pack("<Q", n) for n in ne)
        head += struct.pack("<IQ", t, o)
    start = _align(len(head), alignment)
    blob = bytearray(head + b"\0" * (start - len(head)))
    for (_, _, _, data), o in zip(tensors, rel):
        blob += b"\0" * (start + o - len(blob))
        blob += bytes(data)
    if truncate is not None:
        blob = blob[:truncate]
    with open(path, "wb") as f:
        f.write(blob)
    return {name: start + o for (name, _, _, _), o in zip(tensors, rel)}


def write_split(stem: str, n: int, kvs: Sequence[tuple], tensors: Sequence[tuple]) -> list:
    """Shards stem-0000k-of-0000n.gguf: metadata in the first, tensors dealt out in order."""
    paths, per = [], (len(tensors) + n - 1) // n
    for k in range(n):
        p = f"{stem}-{k + 1:05d}-of-{n:05d}.gguf"
        split_kv = [("split.no", U16, k), ("split.count", U16, n)]
        write_gguf(p, (list(kvs) if k == 0 else []) + split_kv, tensors[k * per:(k + 1) * per])
        paths.append(p)
    return paths


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
