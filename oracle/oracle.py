"""ctypes access to the CPU oracle (liboracle.so) and, where built, the reference (oracle/_ref).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the CPU-baseline
leg of bench.py, always as the checker. The product (large_model_amd) never imports it.
"""
from __future__ import annotations

import ctypes
import os
from typing import Optional, Sequence

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ORACLE_SO = os.path.join(HERE, "liboracle.so")
REF_DIR = os.path.join(HERE, "_ref")

T_F32, T_F16, T_Q4_0, T_Q4_1, T_Q8_0, T_Q6_K = 0, 1, 2, 3, 8, 14
KIND_X, KIND_ROUTER, KIND_GATE, KIND_UP, KIND_DOWN = 0, 1, 2, 3, 4
Q8_DTYPE = np.dtype([("d", "<f4"), ("ds", "<f4"), ("s16", "<i2", (2,)), ("q", "i1", (32,))])

_P = ctypes.c_void_p


class OrcMat(ctypes.Structure):
    _fields_ = [("type", ctypes.c_int), ("rows", ctypes.c_int64), ("cols", ctypes.c_int64),
                ("row_bytes", ctypes.c_uint64), ("expert_bytes", ctypes.c_uint64), ("data", _P)]


class OrcDbg(ctypes.Structure):
    _fields_ = [(n, _P) for n in ("logits", "sel", "wt", "start", "slot_t", "slot_of", "active", "n_active", "xq",
                                  "gu", "act", "aq", "dn")]


def _ptr(a):
    return None if a is None else a.ctypes.data_as(_P)


def _load_oracle():
    if not os.path.exists(ORACLE_SO):
        raise ImportError(f"{ORACLE_SO} missing: run `make -C oracle` (or __graft_entry__.build())")
    L = ctypes.CDLL(ORACLE_SO)
    L.orc_row_bytes.restype = ctypes.c_uint64
    L.orc_row_bytes.argtypes = [ctypes.c_int, ctypes.c_int64]
    L.orc_quantize_q8.argtypes = [_P, ctypes.c_int64, _P]
    L.orc_vec_dot_q8.restype = ctypes.c_float
    L.orc_vec_dot_q8.argtypes = [ctypes.c_int, _P, _P, ctypes.c_int64]
    L.orc_vec_dot_f32.restype = ctypes.c_float
    L.orc_vec_dot_f32.argtypes = [_P, _P, ctypes.c_int64]
    L.orc_block_dot.restype = ctypes.c_int32
    L.orc_block_dot.argtypes = [ctypes.c_int, _P, _P, ctypes.c_int64]
    L.orc_block_dots_at.argtypes = [ctypes.c_int, _P, ctypes.c_uint64, ctypes.c_uint64, ctypes.c_int64, _P, _P, _P, _P,
                                    _P, _P]
    L.orc_matmul_q8.argtypes = [ctypes.c_int, _P, ctypes.c_int64, ctypes.c_int64, ctypes.c_uint64, _P, ctypes.c_int, _P]
    L.orc_dequant_row.argtypes = [ctypes.c_int, _P, _P, ctypes.c_int64]
    L.orc_silu.restype = ctypes.c_float
    L.orc_silu.argtypes = [ctypes.c_float]
    L.orc_f16_to_f32.restype = ctypes.c_float
    L.orc_f16_to_f32.argtypes = [ctypes.c_uint16]
    L.orc_route.argtypes = [ctypes.c_int] * 3 + [_P, _P, ctypes.c_int, _P, _P, _P]
    L.orc_moe.argtypes = [ctypes.c_int] * 4 + [ctypes.POINTER(OrcMat)] * 4 + [_P, ctypes.c_int, _P,
                                                                             ctypes.POINTER(OrcDbg)]
    L.orc_moe_exact.argtypes = L.orc_moe.argtypes
    L.orc_route_exact.argtypes = L.orc_route.argtypes
    L.orc_matmul_exact.argtypes = [ctypes.c_int, _P, ctypes.c_int64, ctypes.c_int64, ctypes.c_uint64, _P,
                                   ctypes.c_int, _P]
    L.orc_synth_f32.argtypes = [ctypes.c_uint64, ctypes.c_uint32, ctypes.c_uint32, ctypes.c_uint32, ctypes.c_uint64,
                                ctypes.c_float, _P]
    L.orc_synth_experts.argtypes = [ctypes.c_uint64, ctypes.c_uint32, ctypes.c_uint32, ctypes.c_int, ctypes.c_int64,
                                    ctypes.c_int64, ctypes.c_int, ctypes.c_int, ctypes.c_float, _P]
    L.orc_rmsnorm_unit.argtypes = [_P, _P, ctypes.c_int, ctypes.c_float]
    L.orc_rmsnorm.argtypes = [_P, _P, _P, ctypes.c_int, ctypes.c_float]
    L.orc_expf_mismatches.restype = ctypes.c_uint64
    L.orc_expf_mismatches.argtypes = [ctypes.c_uint64, ctypes.c_uint64]
    L.orc_exp_mismatches.restype = ctypes.c_uint64
    L.orc_exp_mismatches.argtypes = [ctypes.c_uint64, ctypes.c_int64]
    return L


lib = _load_oracle()


def set_mutation(m: int):
    """Plant one of the oracle's ORC_MUT_* mistakes (0 restores the faithful restatement)."""
    ctypes.c_int.in_dll(lib, "orc_mutation").value = m


def row_bytes(t: int, n: int) -> int:
    return int(lib.orc_row_bytes(t, n))


def quantize_q8(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32).ravel()
    out = np.empty(x.size // 32, Q8_DTYPE)
    lib.orc_quantize_q8(_ptr(x), x.size, _ptr(out))
    return out


def vec_dot_q8(t: int, w: np.ndarray, xq: np.ndarray, n: int) -> float:
    return float(lib.orc_vec_dot_q8(t, _ptr(np.ascontiguousarray(w, np.uint8)), _ptr(xq), n))


def vec_dot_f32(w: np.ndarray, x: np.ndarray) -> float:
    w = np.ascontiguousarray(w, np.float32)
    x = np.ascontiguousarray(x, np.float32)
    return float(lib.orc_vec_dot_f32(_ptr(w), _ptr(x), w.size))


def matmul_q8(t: int, w: np.ndarray, rows: int, cols: int, x: np.ndarray) -> np.ndarray:
    """qms_matmul's fast path (src/quant.c:128-170) for one matrix: y [T][rows]. w holds the
    GGUF row bytes (any dtype; F32 rows may be passed as float32)."""
    x = np.ascontiguousarray(x, np.float32).reshape(-1, cols)
    y = np.empty((x.shape[0], rows), np.float32)
    wb = np.ascontiguousarray(w).reshape(-1).view(np.uint8)
    assert wb.size == rows * row_bytes(t, cols)
    assert lib.orc_matmul_q8(t, _ptr(wb), rows, cols, row_bytes(t, cols), _ptr(x), x.shape[0], _ptr(y)) == 0
    return y


def block_dot(t: int, w_row: np.ndarray, xq: np.ndarray, blk: int) -> int:
    return int(lib.orc_block_dot(t, _ptr(np.ascontiguousarray(w_row, np.uint8)), _ptr(xq), blk))


def block_dots_at(t: int, w: np.ndarray, rb: int, eb: int, ex, row, blk, xq: np.ndarray, xrow) -> np.ndarray:
    """block_dot of stacked expert tensor w at each (expert, row, block) against Q8 row xrow of
    xq (xrow counts Q8 blocks from the start of xq)."""
    ex, row, blk = (np.ascontiguousarray(v, np.int32) for v in (ex, row, blk))
    xrow = np.ascontiguousarray(xrow, np.int64)
    xq = np.ascontiguousarray(xq).reshape(-1)
    assert xq.dtype == Q8_DTYPE and ex.shape == row.shape == blk.shape == xrow.shape
    out = np.empty(ex.shape[0], np.int32)
    lib.orc_block_dots_at(t, _ptr(w), rb, eb, ex.shape[0], _ptr(ex), _ptr(row), _ptr(blk), _ptr(xq), _ptr(xrow),
                          _ptr(out))
    return out


def matmul_exact(t: int, w: np.ndarray, rows: int, cols: int, x: np.ndarray) -> np.ndarray:
    """qms_matmul's matmul_exact (src/quant.c:97-115): dequantised fp32 rows, sequential FMA
    chains. y [T][rows]."""
    x = np.ascontiguousarray(x, np.float32).reshape(-1, cols)
    y = np.empty((x.shape[0], rows), np.float32)
    wb = np.ascontiguousarray(w).reshape(-1).view(np.uint8)
    assert wb.size == rows * row_bytes(t, cols)
    assert lib.orc_matmul_exact(t, _ptr(wb), rows, cols, row_bytes(t, cols), _ptr(x), x.shape[0], _ptr(y)) == 0
    return y


FAST_TYPES = (T_F32, T_Q4_0, T_Q4_1, T_Q6_K)       # qms_fast_supported, src/kernels.c:197-200


def matmul_n(mats, x: np.ndarray, exact: bool = False) -> list:
    """qms_matmul_n (src/quant.c:128-170) on matrices [(type, bytes, rows, cols)] of equal cols:
    the int8 / dot_f32 loop for all of them, unless --exact is set or any one of them is
    outside the fast path (type or cols), which sends every one to matmul_exact (131-141)."""
    fast = not exact and all(t in FAST_TYPES and c % (256 if t == T_Q6_K else 32) == 0 for t, _, _, c in mats)
    fn = matmul_q8 if fast else matmul_exact
    return [fn(t, w, r, c, x) for t, w, r, c in mats]


def dequant_row(t: int, w: np.ndarray, n: int) -> np.ndarray:
    out = np.empty(n, np.float32)
    assert lib.orc_dequant_row(t, _ptr(np.ascontiguousarray(w, np.uint8)), _ptr(out), n) == 0
    return out


def synth_f32(seed: int, layer: int, kind: int, expert: int, n: int, sigma: float) -> np.ndarray:
    out = np.empty(n, np.float32)
    lib.orc_synth_f32(seed, layer, kind, expert, n, sigma, _ptr(out))
    return out


def synth_mat(t: int, rows: int, cols: int, seed: int, sigma: float = 0.02) -> np.ndarray:
    """The GGUF bytes of a seeded synthetic [rows][cols] matrix of type t, as qmsg_mat_synth
    writes them: the expert generator's one 'expert' 0 of kind gate at layer 0 (F32: its normal
    values times sigma)."""
    if t == T_F32:
        return synth_f32(seed, 0, KIND_GATE, 0, rows * cols, sigma).view(np.uint8)
    w = np.zeros(rows * row_bytes(t, cols), np.uint8)
    lib.orc_synth_experts(seed, 0, KIND_GATE, t, rows, cols, 0, 1, sigma, _ptr(w))
    return w


def rmsnorm(x: np.ndarray, w: Optional[np.ndarray] = None, eps: float = 1e-6) -> np.ndarray:
    """Row-wise rmsnorm (src/model.c:403-409); w = None is a unit weight."""
    x = np.ascontiguousarray(x, np.float32).reshape(-1, x.shape[-1])
    wp = None if w is None else np.ascontiguousarray(w, np.float32)
    y = np.empty_like(x)
    for t in range(x.shape[0]):
        lib.orc_rmsnorm(_ptr(y[t]), _ptr(x[t]), _ptr(wp), x.shape[1], eps)
    return y


def rmsnorm_unit(x: np.ndarray, eps: float = 1e-6) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32)
    y = np.empty_like(x)
    for t in range(x.shape[0]):
        lib.orc_rmsnorm_unit(_ptr(y[t]), _ptr(x[t]), x.shape[1], eps)
    return y


class Layer:
    """Host copy of one synthetic layer in GGUF layout (router f32 [X][E], stacked experts)."""

    def __init__(self, E, X, K, F, seed, layer=0, gate_type=T_Q4_0, up_type=T_Q4_0, down_type=T_Q4_0,
                 sigma=0.02, experts: Optional[Sequence[int]] = None, router_col0: Optional[np.ndarray] = None):
        self.E, self.X, self.K, self.F = E, X, K, F
        self.seed, self.layer, self.sigma = seed, layer, sigma
        self.types = (gate_type, up_type, down_type)
        self.router = synth_f32(seed, layer, KIND_ROUTER, 0, X * E, sigma).reshape(X, E)
        if router_col0 is not None:
            self.router[:, 0] = router_col0
        self.rb = (row_bytes(gate_type, E), row_bytes(up_type, E), row_bytes(down_type, F))
        self.eb = (self.rb[0] * F, self.rb[1] * F, self.rb[2] * E)
        # zero-filled (lazily paged) stacks; only requested experts are generated
        self.gate = np.zeros(X * self.eb[0], np.uint8)
        self.up = np.zeros(X * self.eb[1], np.uint8)
        self.down = np.zeros(X * self.eb[2], np.uint8)
        self.have = set()
        self.ensure(range(X) if experts is None else experts)

    def ensure(self, experts):
        for e in sorted(set(int(v) for v in experts) - self.have):
            for kind, t, rows, cols, buf in ((KIND_GATE, self.types[0], self.F, self.E, self.gate),
                                            (KIND_UP, self.types[1], self.F, self.E, self.up),
                                            (KIND_DOWN, self.types[2], self.E, self.F, self.down)):
                lib.orc_synth_experts(self.seed, self.layer, kind, t, rows, cols, e, e + 1, self.sigma, _ptr(buf))
            self.have.add(e)

    def mats(self):
        E, X, F = self.E, self.X, self.F
        r = OrcMat(T_F32, X, E, 4 * E, 4 * E * X, self.router.ctypes.data)
        g = OrcMat(self.types[0], F, E, self.rb[0], self.eb[0], self.gate.ctypes.data)
        u = OrcMat(self.types[1], F, E, self.rb[1], self.eb[1], self.up.ctypes.data)
        d = OrcMat(self.types[2], E, F, self.rb[2], self.eb[2], self.down.ctypes.data)
        return r, g, u, d

    def route(self, xn: np.ndarray, exact: bool = False):
        xn = np.ascontiguousarray(xn, np.float32)
        T = xn.shape[0]
        logits = np.empty((T, self.X), np.float32)
        sel = np.empty((T, self.K), np.int32)
        wt = np.empty((T, self.K), np.float32)
        fn = lib.orc_route_exact if exact else lib.orc_route
        fn(self.E, self.X, self.K, _ptr(self.router), _ptr(xn), T, _ptr(logits), _ptr(sel), _ptr(wt))
        return logits, sel, wt

    def moe(self, xn: np.ndarray, debug: bool = False, exact: bool = False):
        """The oracle layer; returns out, or (out, intermediates) with debug=True. exact: the
        reference's --exact mode (fp32 dequantised rows, no int8)."""
        xn = np.ascontiguousarray(xn, np.float32)
        T = xn.shape[0]
        _, sel, _ = self.route(xn, exact)
        self.ensure(np.unique(sel))
        E, X, K, F = self.E, self.X, self.K, self.F
        NS = T * K
        out = np.empty((T, E), np.float32)
        d = None
        dbg = None
        if debug:
            d = {"logits": np.empty((T, X), np.float32), "sel": np.empty((T, K), np.int32),
                 "wt": np.empty((T, K), np.float32), "start": np.empty(X + 1, np.int32),
                 "slot_t": np.empty(NS, np.int32), "slot_of": np.empty((T, K), np.int32),
                 "active": np.empty(X, np.int32), "n_active": np.empty(1, np.int32),
                 "xq": np.empty((T, E // 32), Q8_DTYPE), "gu": np.empty((NS, 2 * F), np.float32),
                 "act": np.empty((NS, F), np.float32), "aq": np.empty((NS, F // 32), Q8_DTYPE),
                 "dn": np.empty((NS, E), np.float32)}
            dbg = OrcDbg(**{k: v.ctypes.data for k, v in d.items()})
        r, g, u, dm = self.mats()
        fn = lib.orc_moe_exact if exact else lib.orc_moe
        rc = fn(E, X, K, F, ctypes.byref(r), ctypes.byref(g), ctypes.byref(u), ctypes.byref(dm), _ptr(xn), T,
                _ptr(out), ctypes.byref(dbg) if dbg is not None else None)
        if rc != 0:
            raise RuntimeError(f"orc_moe failed ({rc})")
        if debug:
            d["active"] = d["active"][: int(d["n_active"][0])]
            return out, d
        return out


def make_input(E: int, T: int, seed: int, layer: int = 0, sigma: float = 1.0, rmsnorm: bool = False,
               bias_col0: bool = False) -> np.ndarray:
    """The seeded layer input [T][E] (same values as qmsg_synth_input on the device)."""
    x = synth_f32(seed, layer, KIND_X, 0, T * E, sigma).reshape(T, E)
    if rmsnorm:
        x = rmsnorm_unit(x)
    if bias_col0:
        x[:, 0] = 1.0
    return x


# ------------------------------------------------------------------ reference build (oracle/_ref)

def ref_library_path() -> Optional[str]:
    """The reference build for this CPU (VNNI variant when the host has AVX-512 VNNI)."""
    flags = ""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("flags"):
                    flags = line
                    break
    except OSError:
        pass
    names = ["libqms_ref_vnni.so", "libqms_ref_avx2.so"] if ("avx512_vnni" in flags and "avx512vl" in flags) \
        else ["libqms_ref_avx2.so"]
    for n in names:
        p = os.path.join(REF_DIR, n)
        if os.path.exists(p):
            return p
    return None


def load_ref():
    p = ref_library_path()
    if p is None:
        return None
    R = ctypes.CDLL(p)
    R.qref_moe.argtypes = [ctypes.c_int] * 4 + [_P, ctypes.c_int, _P, ctypes.c_int, _P, ctypes.c_int, _P, _P,
                                                 ctypes.c_int, _P]
    R.qms_quantize_q8.argtypes = [_P, ctypes.c_int64, _P]
    R.qms_vec_dot_q8.restype = ctypes.c_float
    R.qms_vec_dot_q8.argtypes = [ctypes.c_int, _P, _P, ctypes.c_int64]
    R.qms_vec_dot_f32.restype = ctypes.c_float
    R.qms_vec_dot_f32.argtypes = [_P, _P, ctypes.c_int64]
    R.qms_dequant_row.argtypes = [ctypes.c_int, _P, _P, ctypes.c_int64]
    R.qref_silu.restype = ctypes.c_float
    R.qref_silu.argtypes = [ctypes.c_float]
    R.qref_rmsnorm_unit.argtypes = [_P, _P, ctypes.c_int, ctypes.c_float]
    R.qref_rmsnorm.argtypes = [_P, _P, _P, ctypes.c_int, ctypes.c_float]
    R.qref_gguf_table.argtypes = [ctypes.c_char_p, ctypes.c_int] + [_P] * 7
    R.qref_gguf_value.argtypes = [ctypes.c_char_p, ctypes.c_char_p, _P, _P]
    R.qref_gguf_moe.argtypes = [ctypes.c_char_p, ctypes.c_int, _P, ctypes.c_int, _P]
    R.qref_isa.restype = ctypes.c_char_p
    R.qref_max_threads.restype = ctypes.c_int
    return R


def ref_moe(R, layer: Layer, xn: np.ndarray, exact: bool = False) -> np.ndarray:
    """The reference's own moe() on the layer; exact sets its qms_exact_math (--exact) for the call."""
    xn = np.ascontiguousarray(xn, np.float32)
    T = xn.shape[0]
    out = np.empty((T, layer.E), np.float32)
    flag = ctypes.c_int.in_dll(R, "qms_exact_math")
    flag.value = 1 if exact else 0
    try:
        rc = R.qref_moe(layer.E, layer.X, layer.K, layer.F, _ptr(layer.router), layer.types[0], _ptr(layer.gate),
                        layer.types[1], _ptr(layer.up), layer.types[2], _ptr(layer.down), _ptr(xn), T, _ptr(out))
    finally:
        flag.value = 0
    if rc != 0:
        raise RuntimeError(f"reference moe() returned {rc}")
    return out
