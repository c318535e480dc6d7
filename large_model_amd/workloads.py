"""Benchmark workloads: the Qwen3-MoE layer shapes the reference is measured on.

Algorithmic work per layer call (what the roofline figures use): bytes = router 4*X*E +
the gate, up and down bytes of every distinct active expert + input and output rows 8*T*E;
int8 operations = 2 * T*K * 3 * E * F. Intermediates are not counted.
"""
from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np

from .qmsg import QMSG_T_Q4_0, QMSG_T_Q6_K, row_bytes

HBM_PEAK_GBS = 8000.0          # MI355X HBM3E, published
INT8_PEAK_TOPS = 5000.0        # MI355X dense int8 MFMA, published (no sparsity)


@dataclass
class Workload:
    name: str
    E: int
    X: int
    K: int
    F: int
    T: int
    seed: int
    down_type: int = QMSG_T_Q4_0
    rmsnorm: bool = False
    zipf: bool = False
    layers: int = 1
    note: str = ""
    extra: dict = field(default_factory=dict)

    @property
    def gate_bytes(self) -> int:          # one expert's gate (= up) matrix
        return row_bytes(QMSG_T_Q4_0, self.E) * self.F

    @property
    def down_bytes(self) -> int:
        return row_bytes(self.down_type, self.F) * self.E

    @property
    def expert_bytes(self) -> int:
        return 2 * self.gate_bytes + self.down_bytes

    def layer_bytes(self, n_active: int) -> int:
        return 4 * self.X * self.E + n_active * self.expert_bytes + 8 * self.T * self.E

    def int8_ops(self) -> int:
        return 2 * self.T * self.K * 3 * self.E * self.F


WORKLOADS = {
    "tiny": Workload("tiny", 256, 16, 4, 128, 1, 0, note="tiny random-init layer, hidden 256, 16 experts top-4"),
    "q30b_decode_t1": Workload("q30b_decode_t1", 2048, 128, 8, 768, 1, 1, rmsnorm=True,
                               note="Qwen3-30B-A3B-shape MoE layer, batch-1 decode"),
    "q235b_decode_t1": Workload("q235b_decode_t1", 4096, 128, 8, 1536, 1, 2,
                                note="Qwen3-235B-A22B-shape MoE layer, batch-1 decode"),
    "q235b_decode_t4": Workload("q235b_decode_t4", 4096, 128, 8, 1536, 4, 2,
                                note="Qwen3-235B-A22B-shape MoE layer, 4-token decode batch"),
    "q235b_decode_t16": Workload("q235b_decode_t16", 4096, 128, 8, 1536, 16, 2,
                                 note="Qwen3-235B-A22B-shape MoE layer, 16-token decode batch"),
    "q235b_prefill_t512": Workload("q235b_prefill_t512", 4096, 128, 8, 1536, 512, 5, zipf=True,
                                   note="Qwen3-235B-A22B-shape MoE layer, 512-token prefill, Zipf(1.1) expert load"),
    "q235b_stack_t64": Workload("q235b_stack_t64", 4096, 128, 8, 1536, 64, 6, down_type=QMSG_T_Q6_K, layers=94,
                                note="Qwen3-235B-A22B-shape 94-layer expert stack, Q6_K down, 64-token decode"),
}


def zipf_targets(X: int, K: int, T: int, s: float = 1.1) -> np.ndarray:
    """Per-expert selection counts proportional to rank^-s, capped at T (top-K picks an
    expert at most once per token) and summing to T*K."""
    w = np.arange(1, X + 1, dtype=np.float64) ** -s
    total = float(T * K)
    c = np.zeros(X)
    free = np.ones(X, bool)
    remaining = total
    for _ in range(X):
        share = remaining * w[free] / w[free].sum()
        over = share > T
        idx = np.flatnonzero(free)
        if not over.any():
            c[idx] = share
            break
        c[idx[over]] = T
        free[idx[over]] = False
        remaining = total - c[~free].sum()
    return c


def zipf_bias(X: int, K: int, T: int, E: int, s: float = 1.1, sigma_w: float = 0.02, iters: int = 300,
              seed: int = 1234) -> np.ndarray:
    """Router bias b (one float per expert, placed in router column 0 while the input's
    column 0 is 1.0) under which the top-K selection counts of T tokens follow Zipf(s).

    Calibrated on an independent Gaussian sample with the logits' spread (the router rows
    are N(0, sigma_w), the inputs N(0, 1)): b_e += log(target_e / count_e) until the counts fit.
    Deterministic: numpy's PCG64 stream for `seed`."""
    rng = np.random.default_rng(seed)
    noise = rng.standard_normal((T, X)) * (sigma_w * np.sqrt(E - 1))
    target = zipf_targets(X, K, T, s)
    b = np.log(target / target.mean())
    step = 0.5
    for _ in range(iters):
        z = noise + b
        top = np.argpartition(-z, K - 1, axis=1)[:, :K]
        cnt = np.bincount(top.ravel(), minlength=X).astype(np.float64)
        b += step * (np.log(target + 0.5) - np.log(cnt + 0.5))
        b -= b.max()
    return b.astype(np.float32)
