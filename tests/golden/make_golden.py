#!/usr/bin/env python3
"""Write the golden vectors under tests/golden/ from the reference's own C code.

Runs in the build container only: it needs oracle/_ref/libqms_ref_*.so, which oracle/Makefile
builds from the reference's sources (src/kernels.c, src/quant.c, src/gguf.c, and src/model.c
through oracle/ref_harness.c). The inputs come from the seeded generator shared with the
device (large_model_amd/csrc/qmsg_synth.h, host copy in the oracle library) and, for the
kernel vectors, from the LCG case generator of the reference's tests/test_kernels.c.

Outputs (numpy .npz, no pickles):
  kat_kernels.npz  qms_quantize_q8 / qms_vec_dot_q8 / qms_vec_dot_f32 / qms_dequant_row
                   results on the test_kernels.c-style cases, plus quantiser tie cases
  layer_*.npz      the reference moe() on whole layers: inputs' hashes, router logits
                   (qms_matmul), int8 input blocks (qms_quantize_q8) and the layer output
  dense.npz        qms_matmul on dense (trunk-shaped) matrices: inputs' hashes and
                   outputs
"""
import ctypes
import hashlib
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, os.path.join(ROOT, "oracle"))
sys.path.insert(0, ROOT)
import oracle as orc  # noqa: E402

P = ctypes.c_void_p


def ptr(a):
    return a.ctypes.data_as(P)


class QmsMat(ctypes.Structure):   # src/quant.h:11-16
    _fields_ = [("type", ctypes.c_int), ("rows", ctypes.c_int64), ("cols", ctypes.c_int64),
                ("row_bytes", ctypes.c_uint64), ("data", P)]


def sha(*arrays) -> str:
    h = hashlib.sha256()
    for a in arrays:
        h.update(np.ascontiguousarray(a).view(np.uint8).tobytes())
    return h.hexdigest()


class Lcg:
    """The case generator of the reference's tests/test_kernels.c:13-14 (seed 12345)."""

    def __init__(self, seed=12345):
        self.s = seed

    def rnd(self) -> int:
        self.s = (self.s * 1664525 + 1013904223) & 0xFFFFFFFF
        return self.s >> 8


def put_f16(w, off, sign, exp, mant):
    h = (sign << 15) | (exp << 10) | mant
    w[off] = h & 0xFF
    w[off + 1] = h >> 8


def fill_block(g: Lcg, t: int, n: int) -> np.ndarray:
    """tests/test_kernels.c:22-39: random bytes with sane fp16 scales."""
    rb = orc.row_bytes(t, n)
    w = np.array([g.rnd() & 0xFF for _ in range(rb)], np.uint8)
    if t in (orc.T_Q4_0, orc.T_Q4_1):
        bs = 18 if t == orc.T_Q4_0 else 20
        for b in range(n // 32):
            put_f16(w, b * bs, 0, 9 + g.rnd() % 4, g.rnd() % 1024)
            if t == orc.T_Q4_1:
                put_f16(w, b * bs + 2, 1, 9 + g.rnd() % 4, g.rnd() % 1024)
    elif t == orc.T_Q6_K:
        for b in range(n // 256):
            for j in range(16):
                w[b * 210 + 192 + j] = np.uint8(np.int8((g.rnd() % 128) - 64))
            put_f16(w, b * 210 + 208, 0, 5 + g.rnd() % 3, g.rnd() % 1024)
    return w


def kat_kernels(R) -> dict:
    out = {}
    g = Lcg()
    cases = []
    for t, sizes in ((orc.T_Q4_0, (256, 1536, 4096)), (orc.T_Q4_1, (256, 1536)), (orc.T_Q6_K, (256, 1536))):
        for n in sizes:
            for trial in range(2):
                w = fill_block(g, t, n)
                x = np.array([((g.rnd() % 20001) - 10000.0) / 3000.0 for _ in range(n)], np.float32)
                if trial == 0:
                    x[:32] = 0.0               # an all-zero block, as test_kernels.c:68 does
                xq = np.empty(n // 32, orc.Q8_DTYPE)
                R.qms_quantize_q8(ptr(x), n, ptr(xq))
                dot = np.float32(R.qms_vec_dot_q8(t, ptr(w), ptr(xq), n))
                deq = np.empty(n, np.float32)
                R.qms_dequant_row(t, ptr(w), ptr(deq), n)
                cases.append((t, n, w, x, xq, dot, deq))
    for i, (t, n, w, x, xq, dot, deq) in enumerate(cases):
        out[f"k{i}_type"] = np.int32(t)
        out[f"k{i}_w"] = w
        out[f"k{i}_x"] = x
        out[f"k{i}_xq"] = xq.view(np.uint8)
        out[f"k{i}_dot"] = np.float32(dot)
        out[f"k{i}_deq_sha"] = np.frombuffer(bytes.fromhex(sha(deq)), np.uint8)
    out["n_kernel_cases"] = np.int32(len(cases))
    # quantiser ties: blocks whose max is 127 (d = 1, 1/d = 1) hold exact halves
    ties = np.zeros(128, np.float32)
    ties[0:32] = np.arange(32) - 15.5
    ties[0] = 127.0
    ties[32:64] = -(np.arange(32) + 0.5)
    ties[32] = -127.0
    ties[64:96] = np.linspace(-3.0, 3.0, 32, dtype=np.float32)
    ties[96:128] = np.float32(1e-30) * np.arange(32)
    tq = np.empty(4, orc.Q8_DTYPE)
    R.qms_quantize_q8(ptr(ties), 128, ptr(tq))
    out["ties_x"] = ties
    out["ties_xq"] = tq.view(np.uint8)
    # fp32 router dot (dot_f32): lengths with and without a 16-element tail
    rng = np.random.default_rng(7)
    for i, n in enumerate((256, 1024, 4096, 4104)):
        w = rng.standard_normal(n).astype(np.float32) * 0.02
        x = rng.standard_normal(n).astype(np.float32)
        out[f"f{i}_w"] = w
        out[f"f{i}_x"] = x
        out[f"f{i}_dot"] = np.float32(R.qms_vec_dot_f32(ptr(w), ptr(x), n))
    out["n_f32_cases"] = np.int32(4)
    # rmsnorm (src/model.c:403-409) around the layer: unit and random weights, varied scales
    for i, (n, scale, unit) in enumerate(((2048, 1.0, True), (4096, 1.0, True), (4096, 37.0, False),
                                           (256, 1e-3, False))):
        x = (rng.standard_normal(n) * scale).astype(np.float32)
        w = np.ones(n, np.float32) if unit else rng.uniform(0.2, 2.0, n).astype(np.float32)
        y = np.empty(n, np.float32)
        R.qref_rmsnorm(ptr(y), ptr(x), ptr(w), n, np.float32(1e-6))
        out[f"r{i}_x"], out[f"r{i}_w"], out[f"r{i}_y"] = x, w, y
    out["n_rms_cases"] = np.int32(4)
    return out


# dense (trunk) matrices through qms_matmul: (type, rows, cols, T, seed)
DENSE = [(orc.T_Q4_0, 512, 4096, 3, 1), (orc.T_Q4_1, 256, 2048, 2, 2), (orc.T_Q4_0, 100, 8192, 1, 3),
         (orc.T_Q4_0, 64, 4096, 9, 4), (orc.T_Q6_K, 96, 4096, 3, 5), (orc.T_Q6_K, 40, 2048, 9, 6),
         (orc.T_F32, 64, 2048, 2, 7), (orc.T_F32, 40, 4096, 6, 8)]


def dense_mat(t, rows, cols, seed):
    return orc.synth_mat(t, rows, cols, seed)


def dense_cases(R) -> dict:
    out = {}
    for i, (t, rows, cols, T, seed) in enumerate(DENSE):
        w = dense_mat(t, rows, cols, seed)
        x = orc.make_input(cols, T, seed)
        y = np.empty((T, rows), np.float32)
        m = QmsMat(t, rows, cols, orc.row_bytes(t, cols), w.ctypes.data)
        R.qms_matmul(ctypes.byref(m), ptr(x), T, ptr(y))
        out[f"d{i}_shape"] = np.array([t, rows, cols, T, seed], np.int64)
        out[f"d{i}_w_sha"] = np.frombuffer(bytes.fromhex(sha(w)), np.uint8)
        out[f"d{i}_x_sha"] = np.frombuffer(bytes.fromhex(sha(x)), np.uint8)
        out[f"d{i}_y"] = y
    out["n_dense_cases"] = np.int32(len(DENSE))
    return out


# name: (E, X, K, F, T, seed, down_type, rmsnorm, special)
LAYERS = {
    "tiny_t1": (256, 16, 4, 128, 1, 0, orc.T_Q4_0, False, None),
    "tiny_t7": (256, 16, 4, 128, 7, 0, orc.T_Q4_0, False, None),
    "tiny_ties": (256, 16, 4, 128, 3, 11, orc.T_Q4_0, False, "ties"),
    "tiny_zero_row": (256, 16, 4, 128, 2, 12, orc.T_Q4_0, False, "zero"),
    "tiny_large": (256, 16, 4, 128, 2, 13, orc.T_Q4_0, False, "large"),
    "q30b_t1": (2048, 128, 8, 768, 1, 1, orc.T_Q4_0, True, None),
    "q235b_t1": (4096, 128, 8, 1536, 1, 2, orc.T_Q4_0, False, None),
    "q235b_t4": (4096, 128, 8, 1536, 4, 2, orc.T_Q4_0, False, None),
    "q235b_t16": (4096, 128, 8, 1536, 16, 2, orc.T_Q4_0, False, None),
    "q235b_q6k_t64": (4096, 128, 8, 1536, 64, 6, orc.T_Q6_K, False, None),
    "q235b_zipf_t512": (4096, 128, 8, 1536, 512, 5, orc.T_Q4_0, False, "zipf"),
    "q235b_q41_t1": (4096, 128, 8, 1536, 1, 7, orc.T_Q4_1, False, None),
    "q235b_q41_t5": (4096, 128, 8, 1536, 5, 7, orc.T_Q4_1, True, None),
    # the widest Qwen3-MoE shape (Qwen3-Coder-480B-A35B: n_embd 6144, 160 experts, n_ff_exp 2560)
    "q480b_t1": (6144, 160, 8, 2560, 1, 12, orc.T_Q4_0, True, None),
    "q480b_t2": (6144, 160, 8, 2560, 2, 13, orc.T_Q4_0, False, None),
    # the reference's --exact mode (qms_exact_math = 1): fp32 dequantised rows, no int8
    "tiny_exact_t3": (256, 16, 4, 128, 3, 30, orc.T_Q4_0, False, "exact"),
    "q30b_exact_t2": (2048, 128, 8, 768, 2, 31, orc.T_Q4_1, True, "exact"),
    "q235b_q6k_exact_t1": (4096, 128, 8, 1536, 1, 32, orc.T_Q6_K, False, "exact"),
    # gate/up other than Q4_0 on the integer path (qms_fast_supported takes any of the three)
    "q30b_gq41_t1": (2048, 128, 8, 768, 1, 33, orc.T_Q4_0, True, None),
    "q235b_gq6k_t4": (4096, 128, 8, 1536, 4, 34, orc.T_Q6_K, False, None),
    "tiny_gq6k_uq41_t7": (256, 16, 4, 128, 7, 35, orc.T_Q4_1, False, None),
}
# gate and up types of the layers above that are not Q4_0 / Q4_0 (stored as "gu_types")
GATE_UP = {
    "q30b_gq41_t1": (orc.T_Q4_1, orc.T_Q4_1),
    "q235b_gq6k_t4": (orc.T_Q6_K, orc.T_Q6_K),
    "tiny_gq6k_uq41_t7": (orc.T_Q6_K, orc.T_Q4_1),
}


def layer_case(R, name, E, X, K, F, T, seed, dt, rms, special):
    col0 = None
    if special == "zipf":
        from large_model_amd.workloads import zipf_bias
        col0 = zipf_bias(X, K, T, E)
    gt, ut = GATE_UP.get(name, (orc.T_Q4_0, orc.T_Q4_0))
    L = orc.Layer(E, X, K, F, seed, gate_type=gt, up_type=ut, down_type=dt, experts=[], router_col0=col0)
    x = orc.make_input(E, T, seed, rmsnorm=rms, bias_col0=special == "zipf")
    if special == "ties":
        L.router[5] = L.router[2]          # experts 2 and 5 tie on every token
        L.router[9] = L.router[2]
    elif special == "zero":
        x[1] = 0.0                         # all logits 0: experts 0..K-1, equal weights
    elif special == "large":
        x *= 300.0
    exact = special == "exact"
    logits, sel, wt = L.route(x, exact)
    L.ensure(np.unique(sel))
    out = orc.ref_moe(R, L, x, exact=exact)
    qm = QmsMat(orc.T_F32, X, E, 4 * E, L.router.ctypes.data)
    ref_logits = np.empty((T, X), np.float32)
    flag = ctypes.c_int.in_dll(R, "qms_exact_math")
    flag.value = int(exact)
    R.qms_matmul(ctypes.byref(qm), ptr(x), T, ptr(ref_logits))
    flag.value = 0
    xq = np.empty((T, E // 32), orc.Q8_DTYPE)
    for t in range(T):
        R.qms_quantize_q8(ptr(x[t]), E, ptr(xq[t]))
    act = np.unique(sel)
    eb = L.eb
    d = {
        "shape": np.array([E, X, K, F, T, seed, dt, int(rms)], np.int64),
        "special": np.array(special or "", dtype="U8"),
        "router_sha": np.frombuffer(bytes.fromhex(sha(L.router)), np.uint8),
        "x_sha": np.frombuffer(bytes.fromhex(sha(x)), np.uint8),
        "experts": act.astype(np.int32),
        "experts_sha": np.frombuffer(bytes.fromhex(sha(*[np.concatenate(
            [L.gate[e * eb[0]:(e + 1) * eb[0]], L.up[e * eb[1]:(e + 1) * eb[1]], L.down[e * eb[2]:(e + 1) * eb[2]]])
            for e in act])), np.uint8),
        "logits_sha": np.frombuffer(bytes.fromhex(sha(ref_logits)), np.uint8),
        "xq_sha": np.frombuffer(bytes.fromhex(sha(xq)), np.uint8),
        "out_sha": np.frombuffer(bytes.fromhex(sha(out)), np.uint8),
    }
    if special == "zipf":
        d["router_col0"] = col0
    if name in GATE_UP:
        d["gu_types"] = np.array([gt, ut], np.int64)
    if out.size <= 16384:
        d["out"] = out
        d["logits"] = ref_logits
    else:
        rng = np.random.default_rng(seed)
        idx = rng.choice(out.size, 256, replace=False)
        d["out_idx"] = idx.astype(np.int64)
        d["out_vals"] = out.ravel()[idx]
    return d


def main():
    R = orc.load_ref()
    if R is None:
        sys.exit("oracle/_ref is not built: run `make -C oracle` where the reference sources are present")
    R.qms_matmul.argtypes = [ctypes.POINTER(QmsMat), P, ctypes.c_int, P]
    print("reference build:", orc.ref_library_path(), R.qref_isa().decode())
    only = sys.argv[1:]                     # optional: regenerate just these files ("dense", layer names)
    if not only:
        np.savez_compressed(os.path.join(HERE, "kat_kernels.npz"), **kat_kernels(R))
    if not only or "dense" in only:
        np.savez_compressed(os.path.join(HERE, "dense.npz"), **dense_cases(R))
        print("wrote dense")
    for name, cfg in LAYERS.items():
        if only and name not in only:
            continue
        d = layer_case(R, name, *cfg)
        np.savez_compressed(os.path.join(HERE, f"layer_{name}.npz"), **d)
        print("wrote", name, "experts", len(d["experts"]))


if __name__ == "__main__":
    main()
