"""Python binding of libqmsg, the MI355X Qwen3-MoE expert-FFN layer.

Mirrors the reference engine's MoE-layer interface (ZeningXiong/large_model):
``moe(m, l, xn, h, T, out)`` (src/model.c:1032) over one layer's ``QmsLayer`` tensors
(src/model.h:37-45) in GGUF layout. ``Context.moe`` has the same argument meaning and the
same error behaviour (a non-zero status raises ``QmsgError`` carrying the library's reason).

The HIP library is required: importing this module on a machine without ``libqmsg.so`` raises
immediately; there is no CPU fallback.
"""
from __future__ import annotations

import ctypes
import os
from typing import Optional

import numpy as np

__all__ = [
    "QMSG_T_F32", "QMSG_T_Q4_0", "QMSG_T_Q4_1", "QMSG_T_Q6_K", "PATH_AUTO", "PATH_EXACT", "PATH_MFMA", "PATH_FP32",
    "Q8_DTYPE", "QmsgError", "Context", "Gguf", "row_bytes", "lib", "library_path",
]

QMSG_T_F32, QMSG_T_F16, QMSG_T_Q4_0, QMSG_T_Q4_1, QMSG_T_Q8_0, QMSG_T_Q6_K = 0, 1, 2, 3, 8, 14
PATH_AUTO, PATH_EXACT, PATH_MFMA, PATH_FP32 = 0, 1, 2, 3

#: QmsQ8 (src/kernels.h:7-12): one int8 activation block of 32 values, 44 bytes.
Q8_DTYPE = np.dtype([("d", "<f4"), ("ds", "<f4"), ("s16", "<i2", (2,)), ("q", "i1", (32,))])
assert Q8_DTYPE.itemsize == 44


def row_bytes(type_: int, ne0: int) -> int:
    """Bytes of one row of ``ne0`` elements (qms_row_bytes, src/gguf.c:85-96); 0 if invalid."""
    if type_ == QMSG_T_F32:
        return ne0 * 4
    if type_ == QMSG_T_F16:
        return ne0 * 2
    if type_ == QMSG_T_Q4_0:
        return 0 if ne0 % 32 else ne0 // 32 * 18
    if type_ == QMSG_T_Q4_1:
        return 0 if ne0 % 32 else ne0 // 32 * 20
    if type_ == QMSG_T_Q8_0:
        return 0 if ne0 % 32 else ne0 // 32 * 34
    if type_ == QMSG_T_Q6_K:
        return 0 if ne0 % 256 else ne0 // 256 * 210
    return 0


class _Mat(ctypes.Structure):
    _fields_ = [("type", ctypes.c_int), ("rows", ctypes.c_int64), ("cols", ctypes.c_int64),
                ("row_bytes", ctypes.c_uint64), ("data", ctypes.c_void_p)]


class _Experts(ctypes.Structure):
    _fields_ = [("m", _Mat), ("expert_bytes", ctypes.c_uint64)]


class _Layer(ctypes.Structure):
    _fields_ = [("router", _Mat), ("gate", _Experts), ("up", _Experts), ("down", _Experts)]


class _Cfg(ctypes.Structure):
    _fields_ = [("n_embd", ctypes.c_int), ("n_expert", ctypes.c_int), ("n_used", ctypes.c_int),
                ("n_ff_exp", ctypes.c_int)]


class _Tensor(ctypes.Structure):
    _fields_ = [("name", ctypes.c_char * 96), ("type", ctypes.c_int), ("n_dims", ctypes.c_int),
                ("ne", ctypes.c_int64 * 4), ("shard", ctypes.c_int), ("off", ctypes.c_uint64),
                ("nbytes", ctypes.c_uint64)]


class _Debug(ctypes.Structure):
    _fields_ = [(n, ctypes.c_void_p) for n in
                ("logits", "sel", "wt", "start", "slot_t", "slot_of", "active", "n_active", "xq", "gu", "act",
                 "aq", "dn")]


_P = ctypes.c_void_p
_I = ctypes.c_int
_SIGS = {
    "qmsg_create": (_I, [ctypes.POINTER(_P), _I, ctypes.POINTER(_Cfg), _I, _I]),
    "qmsg_destroy": (None, [_P]),
    "qmsg_last_error": (ctypes.c_char_p, [_P]),
    "qmsg_stream": (_P, [_P]),
    "qmsg_set_path": (_I, [_P, _I]),
    "qmsg_layer_upload": (_I, [_P, _I, ctypes.POINTER(_Layer)]),
    "qmsg_layer_synth": (_I, [_P, _I, ctypes.c_uint64, _I, _I, _I, ctypes.c_float, _P]),
    "qmsg_layer_download": (_I, [_P, _I, _P, _P, _P, _P]),
    "qmsg_moe": (_I, [_P, _I, _P, _P, _I, _P]),
    "qmsg_moe_device": (_I, [_P, _I, _P, _I, _P]),
    "qmsg_moe_device_noalloc": (_I, [_P, _I, _P, _I, _P]),
    "qmsg_sync": (_I, [_P]),
    "qmsg_device_alloc": (_P, [_P, ctypes.c_size_t]),
    "qmsg_memcpy_h2d": (_I, [_P, _P, _P, ctypes.c_size_t]),
    "qmsg_memcpy_d2h": (_I, [_P, _P, _P, ctypes.c_size_t]),
    "qmsg_synth_input": (_I, [_P, ctypes.c_uint64, _I, _I, ctypes.c_float, _I, _I, _P]),
    "qmsg_moe_debug": (_I, [_P, _I, _P, _I, _P, ctypes.POINTER(_Debug)]),
    "qmsg_block_dots": (_I, [_P, _I, _I, _I, _P, _P, _P, _P, _P]),
    "qmsg_profile": (_I, [_P, _I]),
    "qmsg_profile_read": (_I, [_P, ctypes.c_char_p, ctypes.POINTER(ctypes.c_int64),
                               ctypes.POINTER(ctypes.c_double)]),
    "qmsg_moe_chain": (_I, [_P, _I, _I, _P, _I, ctypes.c_float]),
    "qmsg_rmsnorm_device": (_I, [_P, _P, _P, _P, _I, _I, ctypes.c_float]),
    "qmsg_rmsnorm_mode": (_I, [_P, _I, ctypes.POINTER(ctypes.c_int64)]),
    "qmsg_layer_norm": (_I, [_P, _I, _P]),
    "qmsg_eval_silu": (_I, [_P, _P, _I, _P]),
    "qmsg_eval_exp": (_I, [_P, _P, _I, _P]),
    "qmsg_calibrate_copy": (_I, [_P, _P, _P, ctypes.c_size_t]),
    "qmsg_gguf_open": (_I, [ctypes.POINTER(_P), ctypes.c_char_p]),
    "qmsg_gguf_close": (None, [_P]),
    "qmsg_gguf_n_tensors": (_I, [_P]),
    "qmsg_gguf_tensor": (_I, [_P, _I, ctypes.POINTER(_Tensor)]),
    "qmsg_gguf_find": (_I, [_P, ctypes.c_char_p]),
    "qmsg_gguf_get_int": (_I, [_P, ctypes.c_char_p, ctypes.POINTER(ctypes.c_int64)]),
    "qmsg_gguf_get_float": (_I, [_P, ctypes.c_char_p, ctypes.POINTER(ctypes.c_double)]),
    "qmsg_gguf_get_str": (_I, [_P, ctypes.c_char_p, ctypes.c_char_p, ctypes.c_size_t]),
    "qmsg_gguf_moe_cfg": (_I, [_P, ctypes.POINTER(_Cfg), ctypes.POINTER(_I), ctypes.POINTER(ctypes.c_float)]),
    "qmsg_gguf_upload": (_I, [_P, _P, _I, _I]),
    "qmsg_mat_upload": (_I, [_P, ctypes.POINTER(_Mat), ctypes.POINTER(_I)]),
    "qmsg_gguf_upload_mat": (_I, [_P, _P, ctypes.c_char_p, ctypes.POINTER(_I)]),
    "qmsg_mat_synth": (_I, [_P, _I, ctypes.c_int64, ctypes.c_int64, ctypes.c_uint64, ctypes.c_float,
                            ctypes.POINTER(_I)]),
    "qmsg_matmul_n": (_I, [_P, _P, _I, _P, _I, _P]),
    "qmsg_matmul_n_device": (_I, [_P, _P, _I, _P, _I, _P]),
    "qmsg_device_info": (_I, [_P, ctypes.POINTER(_I), ctypes.POINTER(_I), ctypes.POINTER(ctypes.c_uint64),
                              ctypes.c_char_p, _I]),
}

library_path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libqmsg.so")


def _load() -> ctypes.CDLL:
    if not os.path.exists(library_path):
        raise ImportError(f"libqmsg.so is not built ({library_path}); run __graft_entry__.build() first")
    lib_ = ctypes.CDLL(library_path)
    for name, (res, args) in _SIGS.items():
        fn = getattr(lib_, name)
        fn.restype = res
        fn.argtypes = args
    return lib_


lib = _load()


class QmsgError(RuntimeError):
    def __init__(self, status: int, msg: str):
        super().__init__(f"qmsg status {status}: {msg}")
        self.status = status


def _ptr(a: Optional[np.ndarray]):
    return None if a is None else a.ctypes.data_as(_P)


class Gguf:
    """A parsed GGUF v3 model (qms_gguf_open, src/gguf.c:222-241): tensor table and the first
    shard's scalar metadata. Needs no GPU; ``Context.load_gguf`` moves its MoE tensors to HBM."""

    def __init__(self, path: str):
        h = _P()
        st = lib.qmsg_gguf_open(ctypes.byref(h), os.fsencode(path))
        if st != 0:
            raise QmsgError(st, lib.qmsg_last_error(None).decode())
        self._h = h
        self.path = path

    def close(self):
        if getattr(self, "_h", None):
            lib.qmsg_gguf_close(self._h)
            self._h = None

    def __del__(self):
        self.close()

    def __enter__(self):
        return self

    def __exit__(self, *a):
        self.close()

    def _raise(self, st: int):
        raise QmsgError(st, lib.qmsg_last_error(None).decode())

    def tensors(self) -> list:
        """The tensor table: dicts of name, type, n_dims, ne (4 ints), shard, off, nbytes."""
        out = []
        t = _Tensor()
        for i in range(lib.qmsg_gguf_n_tensors(self._h)):
            st = lib.qmsg_gguf_tensor(self._h, i, ctypes.byref(t))
            if st != 0:
                self._raise(st)
            out.append({"name": t.name.decode(), "type": t.type, "n_dims": t.n_dims, "ne": list(t.ne),
                        "shard": t.shard, "off": t.off, "nbytes": t.nbytes})
        return out

    def find(self, name: str) -> int:
        return lib.qmsg_gguf_find(self._h, name.encode())

    def get_int(self, key: str) -> int:
        v = ctypes.c_int64()
        st = lib.qmsg_gguf_get_int(self._h, key.encode(), ctypes.byref(v))
        if st != 0:
            self._raise(st)
        return v.value

    def get_float(self, key: str) -> float:
        v = ctypes.c_double()
        st = lib.qmsg_gguf_get_float(self._h, key.encode(), ctypes.byref(v))
        if st != 0:
            self._raise(st)
        return v.value

    def get_str(self, key: str) -> str:
        buf = ctypes.create_string_buffer(512)
        st = lib.qmsg_gguf_get_str(self._h, key.encode(), buf, len(buf))
        if st != 0:
            self._raise(st)
        return buf.value.decode()

    def moe_cfg(self) -> dict:
        """read_cfg's MoE keys (src/model.c:278-310): n_embd, n_expert, n_used, n_ff_exp,
        n_layer, eps."""
        cfg, nl, eps = _Cfg(), _I(), ctypes.c_float()
        st = lib.qmsg_gguf_moe_cfg(self._h, ctypes.byref(cfg), ctypes.byref(nl), ctypes.byref(eps))
        if st != 0:
            self._raise(st)
        return {"n_embd": cfg.n_embd, "n_expert": cfg.n_expert, "n_used": cfg.n_used, "n_ff_exp": cfg.n_ff_exp,
                "n_layer": nl.value, "eps": eps.value}


class Context:
    """One device context: resident layers of one shape and scratch for up to ``max_tokens``."""

    def __init__(self, n_embd: int, n_expert: int, n_used: int, n_ff_exp: int, n_layer: int = 1,
                 max_tokens: int = 16, device: int = 0):
        self.E, self.X, self.K, self.F = n_embd, n_expert, n_used, n_ff_exp
        self.n_layer, self.max_tokens = n_layer, max_tokens
        cfg = _Cfg(n_embd, n_expert, n_used, n_ff_exp)
        h = _P()
        st = lib.qmsg_create(ctypes.byref(h), device, ctypes.byref(cfg), n_layer, max_tokens)
        if st != 0:
            raise QmsgError(st, lib.qmsg_last_error(None).decode())
        self._h = h
        self._types = {}

    def close(self):
        if getattr(self, "_h", None):
            lib.qmsg_destroy(self._h)
            self._h = None

    def __del__(self):
        self.close()

    def __enter__(self):
        return self

    def __exit__(self, *a):
        self.close()

    def _check(self, st: int):
        if st != 0:
            raise QmsgError(st, lib.qmsg_last_error(self._h).decode())

    # ---------------------------------------------------------------- weights
    def upload(self, layer: int, router: np.ndarray, gate: tuple, up: tuple, down: tuple):
        """Copy GGUF tensor bytes to HBM: router f32 [X][E]; gate/up/down = (type, uint8 bytes)."""
        E, X, F = self.E, self.X, self.F
        router = np.ascontiguousarray(router, dtype=np.float32)
        L = _Layer()
        L.router = _Mat(QMSG_T_F32, X, E, 4 * E, router.ctypes.data)
        keep = [router]
        for name, (t, buf), rows, cols in (("gate", gate, F, E), ("up", up, F, E), ("down", down, E, F)):
            buf = np.ascontiguousarray(buf, dtype=np.uint8)
            keep.append(buf)
            rb = row_bytes(t, cols)
            getattr(L, name).m = _Mat(t, rows, cols, rb, buf.ctypes.data)
            getattr(L, name).expert_bytes = rb * rows
        self._check(lib.qmsg_layer_upload(self._h, layer, ctypes.byref(L)))
        self._types[layer] = (gate[0], up[0], down[0])

    def synth(self, layer: int, seed: int, gate_type: int = QMSG_T_Q4_0, up_type: int = QMSG_T_Q4_0,
              down_type: int = QMSG_T_Q4_0, sigma: float = 0.02, router_col0: Optional[np.ndarray] = None):
        """Generate the seeded synthetic layer directly in HBM."""
        col = None if router_col0 is None else np.ascontiguousarray(router_col0, dtype=np.float32)
        self._check(lib.qmsg_layer_synth(self._h, layer, seed, gate_type, up_type, down_type, sigma, _ptr(col)))
        self._types[layer] = (gate_type, up_type, down_type)

    def download(self, layer: int):
        """Return (router, gate, up, down) host copies of a resident layer."""
        gt, ut, dt = self._types[layer]
        E, X, F = self.E, self.X, self.F
        router = np.empty((X, E), np.float32)
        gate = np.empty(X * F * row_bytes(gt, E), np.uint8)
        up = np.empty(X * F * row_bytes(ut, E), np.uint8)
        down = np.empty(X * E * row_bytes(dt, F), np.uint8)
        self._check(lib.qmsg_layer_download(self._h, layer, _ptr(router), _ptr(gate), _ptr(up), _ptr(down)))
        return router, gate, up, down

    def load_gguf(self, g: Gguf, first: int = 0, n: Optional[int] = None):
        """Copy file layers first .. first+n-1 (router, gate/up/down experts, ffn_norm) of a
        parsed GGUF into the context's layers of the same index."""
        n = self.n_layer - first if n is None else n
        self._check(lib.qmsg_gguf_upload(self._h, g._h, first, n))
        for t in g.tensors():
            parts = t["name"].split(".")
            if len(parts) == 4 and parts[0] == "blk" and parts[2] in ("ffn_gate_exps", "ffn_up_exps", "ffn_down_exps"):
                layer = int(parts[1])
                if first <= layer < first + n:
                    types = list(self._types.get(layer, (QMSG_T_Q4_0,) * 3))
                    types[("ffn_gate_exps", "ffn_up_exps", "ffn_down_exps").index(parts[2])] = t["type"]
                    self._types[layer] = tuple(types)

    @classmethod
    def from_gguf(cls, g: Gguf, max_tokens: int = 16, device: int = 0) -> "Context":
        """A context shaped by the file's MoE config with every layer loaded."""
        c = g.moe_cfg()
        ctx = cls(c["n_embd"], c["n_expert"], c["n_used"], c["n_ff_exp"], n_layer=c["n_layer"],
                  max_tokens=max_tokens, device=device)
        ctx.eps = c["eps"]
        ctx.load_gguf(g, 0, c["n_layer"])
        return ctx

    # ---------------------------------------------------------------- dense (trunk) products
    def mat_upload(self, type_: int, data: np.ndarray, rows: int, cols: int) -> int:
        """A dense matrix (GGUF rows, QmsMat) resident in HBM; returns its id. data holds the
        row bytes (F32 rows may be given as float32)."""
        data = np.ascontiguousarray(data).reshape(-1).view(np.uint8)
        m = _Mat(type_, rows, cols, row_bytes(type_, cols), data.ctypes.data)
        i = _I()
        self._check(lib.qmsg_mat_upload(self._h, ctypes.byref(m), ctypes.byref(i)))
        self._mats = getattr(self, "_mats", {})
        self._mats[i.value] = (rows, cols)
        return i.value

    def mat_synth(self, type_: int, rows: int, cols: int, seed: int, sigma: float = 0.02) -> int:
        """A resident matrix of seeded synthetic rows generated on the device; returns its id."""
        i = _I()
        self._check(lib.qmsg_mat_synth(self._h, type_, rows, cols, seed, sigma, ctypes.byref(i)))
        self._mats = getattr(self, "_mats", {})
        self._mats[i.value] = (rows, cols)
        return i.value

    def gguf_upload_mat(self, g: "Gguf", name: str) -> int:
        i = _I()
        self._check(lib.qmsg_gguf_upload_mat(self._h, g._h, name.encode(), ctypes.byref(i)))
        t = g.tensors()[g.find(name)]
        self._mats = getattr(self, "_mats", {})
        self._mats[i.value] = (t["ne"][1], t["ne"][0])
        return i.value

    def matmul_n(self, ids, x: np.ndarray) -> list:
        """qms_matmul_n: [y_i [T][rows_i]] for resident matrices ids on host rows x [T][cols]."""
        mats = getattr(self, "_mats", {})
        if any(i not in mats for i in ids):         # let the library report the bad id
            idv = (_I * len(ids))(*ids)
            self._check(lib.qmsg_matmul_n(self._h, idv, len(ids), None, 0, (_P * len(ids))()))
        cols = mats[ids[0]][1]
        x = np.ascontiguousarray(x, np.float32).reshape(-1, cols)
        T = x.shape[0]
        ys = [np.empty((T, self._mats[i][0]), np.float32) for i in ids]
        idv = (_I * len(ids))(*ids)
        yp = (_P * len(ids))(*[y.ctypes.data for y in ys])
        self._check(lib.qmsg_matmul_n(self._h, idv, len(ids), _ptr(x), T, yp))
        return ys

    def matmul_n_device(self, ids, d_x: int, T: int, d_ys):
        idv = (_I * len(ids))(*ids)
        yp = (_P * len(ids))(*d_ys)
        self._check(lib.qmsg_matmul_n_device(self._h, idv, len(ids), d_x, T, yp))

    def set_path(self, path: int):
        self._check(lib.qmsg_set_path(self._h, path))

    # ---------------------------------------------------------------- the layer
    def moe(self, layer: int, xn: np.ndarray, h: Optional[np.ndarray] = None) -> np.ndarray:
        """out[T][E] for xn[T][E] (moe(m, l, xn, h, T, out), src/model.c:1032)."""
        xn = np.ascontiguousarray(xn, dtype=np.float32).reshape(-1, self.E)
        out = np.empty_like(xn)
        self._check(lib.qmsg_moe(self._h, layer, _ptr(xn), None, xn.shape[0], _ptr(out)))
        return out

    def moe_debug(self, layer: int, xn: np.ndarray):
        """Run the layer and return (out, intermediates dict) for parity checks."""
        xn = np.ascontiguousarray(xn, dtype=np.float32).reshape(-1, self.E)
        T, E, X, K, F = xn.shape[0], self.E, self.X, self.K, self.F
        NS = T * K
        d = {
            "logits": np.empty((T, X), np.float32), "sel": np.empty((T, K), np.int32),
            "wt": np.empty((T, K), np.float32), "start": np.empty(X + 1, np.int32),
            "slot_t": np.empty(NS, np.int32), "slot_of": np.empty((T, K), np.int32),
            "active": np.empty(X, np.int32), "n_active": np.empty(1, np.int32),
            "xq": np.empty((T, E // 32), Q8_DTYPE), "gu": np.empty((NS, 2 * F), np.float32),
            "act": np.empty((NS, F), np.float32), "aq": np.empty((NS, F // 32), Q8_DTYPE),
            "dn": np.empty((NS, E), np.float32),
        }
        g = _Debug(**{k: v.ctypes.data for k, v in d.items()})
        out = np.empty_like(xn)
        self._check(lib.qmsg_moe_debug(self._h, layer, _ptr(xn), T, _ptr(out), ctypes.byref(g)))
        d["active"] = d["active"][: int(d["n_active"][0])]
        return out, d

    def block_dots(self, layer: int, which: int, expert, row, block, xq_blocks: np.ndarray) -> np.ndarray:
        """Exact int32 dots of (expert, row, 32-block) weight blocks with QmsQ8 blocks."""
        expert = np.ascontiguousarray(expert, np.int32)
        row = np.ascontiguousarray(row, np.int32)
        block = np.ascontiguousarray(block, np.int32)
        xq_blocks = np.ascontiguousarray(xq_blocks, Q8_DTYPE)
        out = np.empty(expert.shape[0], np.int32)
        self._check(lib.qmsg_block_dots(self._h, layer, which, expert.shape[0], _ptr(expert), _ptr(row),
                                        _ptr(block), _ptr(xq_blocks), _ptr(out)))
        return out

    # ---------------------------------------------------------------- device buffers / timing
    def device_alloc(self, nbytes: int) -> int:
        p = lib.qmsg_device_alloc(self._h, nbytes)
        if not p:
            raise QmsgError(-3, lib.qmsg_last_error(self._h).decode())
        return p

    def synth_input(self, seed: int, layer: int, T: int, d_x: int, sigma: float = 1.0, rmsnorm: bool = False,
                    bias_col0: bool = False):
        self._check(lib.qmsg_synth_input(self._h, seed, layer, T, sigma, int(rmsnorm), int(bias_col0), d_x))

    def moe_device(self, layer: int, d_xn: int, T: int, d_out: int):
        self._check(lib.qmsg_moe_device(self._h, layer, d_xn, T, d_out))

    def moe_device_noalloc(self, layer: int, d_xn: int, T: int, d_out: int):
        """The same layer with the library's static scratch (allocates nothing)."""
        self._check(lib.qmsg_moe_device_noalloc(self._h, layer, d_xn, T, d_out))

    def moe_chain(self, first: int, n: int, d_h: int, T: int, eps: float = 1e-6):
        """h += moe(l, rmsnorm(h, ffn_norm_l)) for layers first .. first+n-1 on device rows d_h."""
        self._check(lib.qmsg_moe_chain(self._h, first, n, d_h, T, eps))

    def rmsnorm_device(self, d_y: int, d_x: int, d_w: Optional[int], rows: int, n: int, eps: float = 1e-6):
        """d_y = rmsnorm(d_x, d_w) row by row on device buffers (d_w None: unit weights)."""
        self._check(lib.qmsg_rmsnorm_device(self._h, d_y, d_x, d_w, rows, n, eps))

    def rmsnorm(self, x: np.ndarray, w: Optional[np.ndarray] = None, eps: float = 1e-6,
                inplace: bool = True) -> np.ndarray:
        """rmsnorm of host rows x [rows][n] on the device (src/model.c:403-409); returns y.
        inplace=False writes y to a buffer of its own and checks that x is left as it was."""
        x = np.ascontiguousarray(x, np.float32)
        rows, n = x.shape
        d_x = self.device_alloc(max(x.nbytes, 16))
        d_y = d_x if inplace else self.device_alloc(max(x.nbytes, 16))
        d_w = None
        self.h2d(d_x, x)
        if w is not None:
            d_w = self.device_alloc(n * 4)
            self.h2d(d_w, np.ascontiguousarray(w, np.float32))
        self.rmsnorm_device(d_y, d_x, d_w, rows, n, eps)
        self.sync()
        if not inplace and not np.array_equal(self.d2h(d_x, (rows, n)).view(np.uint32), x.view(np.uint32)):
            raise QmsgError(-4, "rmsnorm: the input rows changed")
        return self.d2h(d_y, (rows, n))

    def rmsnorm_mode(self, always_walk: bool) -> int:
        """Set how rmsnorm forms its sum (True: in order for every row; False: only for rows the
        parallel bracket leaves open); returns the rows that formed it in order since the last
        call."""
        n = ctypes.c_int64(0)
        self._check(lib.qmsg_rmsnorm_mode(self._h, int(always_walk), ctypes.byref(n)))
        return int(n.value)

    def layer_norm(self, layer: int, w: Optional[np.ndarray]):
        wp = None if w is None else np.ascontiguousarray(w, np.float32)
        self._check(lib.qmsg_layer_norm(self._h, layer, _ptr(wp)))

    def sync(self):
        self._check(lib.qmsg_sync(self._h))

    def d2h(self, d_src: int, shape, dtype=np.float32) -> np.ndarray:
        a = np.empty(shape, dtype)
        self._check(lib.qmsg_memcpy_d2h(self._h, _ptr(a), d_src, a.nbytes))
        return a

    def h2d(self, d_dst: int, a: np.ndarray):
        a = np.ascontiguousarray(a)
        self._check(lib.qmsg_memcpy_h2d(self._h, d_dst, _ptr(a), a.nbytes))

    def profile(self, enable: bool):
        self._check(lib.qmsg_profile(self._h, int(enable)))

    def profile_read(self, name: str):
        n = ctypes.c_int64()
        ms = ctypes.c_double()
        self._check(lib.qmsg_profile_read(self._h, name.encode(), ctypes.byref(n), ctypes.byref(ms)))
        return n.value, ms.value

    def eval_silu(self, x: np.ndarray) -> np.ndarray:
        x = np.ascontiguousarray(x, np.float32).ravel()
        out = np.empty_like(x)
        self._check(lib.qmsg_eval_silu(self._h, _ptr(x), x.size, _ptr(out)))
        return out

    def eval_exp(self, x: np.ndarray) -> np.ndarray:
        x = np.ascontiguousarray(x, np.float64).ravel()
        out = np.empty_like(x)
        self._check(lib.qmsg_eval_exp(self._h, _ptr(x), x.size, _ptr(out)))
        return out

    def calibrate_copy(self, d_dst: int, d_src: int, nbytes: int):
        self._check(lib.qmsg_calibrate_copy(self._h, d_dst, d_src, nbytes))

    def device_info(self) -> dict:
        cu, clk = ctypes.c_int(), ctypes.c_int()
        hbm = ctypes.c_uint64()
        arch = ctypes.create_string_buffer(64)
        self._check(lib.qmsg_device_info(self._h, ctypes.byref(cu), ctypes.byref(clk), ctypes.byref(hbm), arch, 64))
        return {"n_cu": cu.value, "clock_khz": clk.value, "hbm_bytes": hbm.value, "arch": arch.value.decode()}
