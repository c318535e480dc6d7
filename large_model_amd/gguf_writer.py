"""Writing GGUF v3 files (for tests and load-rate measurements; the library itself only reads).

The layout follows the published GGUF v3 format: magic "GGUF", u32 version, u64 tensor count,
u64 metadata count, metadata (string key, u32 value type, value), tensor infos (string name,
u32 n_dims, u64 ne[n_dims], u32 type, u64 offset relative to the data section), padding to
``general.alignment`` (32 unless given), then the tensor data, each tensor at an aligned
offset. Little-endian throughout. Tensor data are written in a stream, so multi-GB files need
no copy in memory.
"""
from __future__ import annotations

import struct
from typing import Optional, Sequence

import numpy as np

U8, I8, U16, I16, U32, I32, F32, BOOL, STR, ARR, U64, I64, F64 = range(13)
_FMT = {U8: "<B", I8: "<b", U16: "<H", I16: "<h", U32: "<I", I32: "<i", F32: "<f", BOOL: "<B",
        U64: "<Q", I64: "<q", F64: "<d"}


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


def _nbytes(data) -> int:
    return data if isinstance(data, int) else len(memoryview(data).cast("B"))


def write_gguf(path: str, kvs: Sequence[tuple], tensors: Sequence[tuple], alignment: int = 32,
               version: int = 3, truncate: Optional[int] = None) -> dict:
    """kvs: (key, value type, value); tensors: (name, ggml type, ne list, data), where data is
    bytes-like or an int n (n bytes of a fixed pseudo-random pattern).
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
        off += _nbytes(data)
    for (name, t, ne, _), o in zip(tensors, rel):
        head += _s(name) + struct.pack("<I", len(ne)) + b"".join(struct.pack("<Q", n) for n in ne)
        head += struct.pack("<IQ", t, o)
    start = _align(len(head), alignment)
    pattern = None
    with open(path, "wb") as f:
        pos = 0

        def put(b):
            nonlocal pos
            b = memoryview(b).cast("B")
            if truncate is not None:
                b = b[:max(0, truncate - pos)]
            f.write(b)
            pos += len(b)

        put(head + b"\0" * (start - len(head)))
        for (_, _, _, data), o in zip(tensors, rel):
            put(b"\0" * (start + o - pos))
            if isinstance(data, int):
                if pattern is None:
                    pattern = np.random.default_rng(1).integers(0, 256, 1 << 22, dtype=np.uint8).tobytes()
                for a in range(0, data, len(pattern)):
                    put(pattern[:min(len(pattern), data - a)])
            else:
                put(data)
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


def moe_header(E: int, X: int, K: int, F: int, n_layer: int, eps: float = 1e-6) -> list:
    """The qwen3moe metadata read_cfg needs (src/model.c:278-310), attention sizes of the 235B
    model (64 query heads, 4 KV heads of 128)."""
    return [
        ("general.architecture", STR, "qwen3moe"),
        ("general.alignment", U32, 32),
        ("qwen3moe.block_count", U32, n_layer),
        ("qwen3moe.embedding_length", U32, E),
        ("qwen3moe.attention.head_count", U32, 64),
        ("qwen3moe.attention.head_count_kv", U32, 4),
        ("qwen3moe.attention.key_length", U32, 128),
        ("qwen3moe.expert_count", U32, X),
        ("qwen3moe.expert_used_count", U32, K),
        ("qwen3moe.expert_feed_forward_length", U32, F),
        ("qwen3moe.attention.layer_norm_rms_epsilon", F32, eps),
        ("qwen3moe.rope.freq_base", F32, 5000000.0),
    ]
