"""Layers whose expert tensors are of any type the reference's loader takes (load_experts,
src/model.c:133-157): Q4_0, Q4_1 and Q6_K from the seeded expert generator, and Q8_0, F16 and
F32 (outside the integer fast path, src/kernels.c:197-200) from seeded numpy draws of the GGUF
block layouts. The reference runs layers with such tensors through moe_group_exact, whose
per-slot qms_matmul picks each matrix's dot by its type (src/model.c:1009-1030, 1090-1093)."""
from __future__ import annotations

import numpy as np

import oracle as orc

GENERATED = (orc.T_Q4_0, orc.T_Q4_1, orc.T_Q6_K)


def expert_bytes(t: int, rows: int, cols: int, X: int, seed: int) -> np.ndarray:
    """GGUF bytes of a stacked [X][rows][cols] expert tensor of type t."""
    if t in GENERATED:
        return orc.synth_mat(t, rows * X, cols, seed)
    rng = np.random.default_rng(seed)
    n = rows * X * cols
    if t == orc.T_F32:
        return (rng.standard_normal(n).astype(np.float32) * np.float32(0.05)).view(np.uint8)
    if t == orc.T_F16:
        return (rng.standard_normal(n) * 0.05).astype(np.float16).view(np.uint8)
    if t == orc.T_Q8_0:                       # { f16 d; i8 q[32] } per 32 elements
        nb = n // 32
        blk = np.empty((nb, 34), np.uint8)
        d = (np.abs(rng.standard_normal(nb)) * 2e-3 + 1e-4).astype(np.float16)
        blk[:, :2] = d.view(np.uint8).reshape(nb, 2)
        blk[:, 2:] = rng.integers(-127, 128, (nb, 32)).astype(np.int8).view(np.uint8)
        return blk.reshape(-1)
    raise ValueError(f"type {t}")


def typed_layer(E: int, X: int, K: int, F: int, types, seed: int) -> orc.Layer:
    """An oracle layer (seeded router) whose gate, up and down stacks hold expert_bytes."""
    gt, ut, dt = types
    L = orc.Layer(E, X, K, F, seed, gate_type=gt, up_type=ut, down_type=dt, experts=[])
    L.gate[:] = expert_bytes(gt, F, E, X, seed + 1)
    L.up[:] = expert_bytes(ut, F, E, X, seed + 2)
    L.down[:] = expert_bytes(dt, E, F, X, seed + 3)
    L.have = set(range(X))
    return L
