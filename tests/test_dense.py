"""Dense (trunk) products on the CPU: the oracle's qms_matmul restatement against the reference's
own qms_matmul outputs (tests/golden/dense.npz) and, where the reference build is present,
live on further shapes."""
import ctypes
import hashlib
import os

import numpy as np
import pytest

import oracle as orc

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def sha(a) -> bytes:
    return hashlib.sha256(np.ascontiguousarray(a).view(np.uint8).tobytes()).digest()


def dense_mat(t, rows, cols, seed):
    return orc.synth_mat(t, rows, cols, seed)


def test_oracle_matmul_matches_reference_fixtures():
    d = dict(np.load(os.path.join(GOLD, "dense.npz")))
    for i in range(int(d["n_dense_cases"])):
        t, rows, cols, T, seed = (int(v) for v in d[f"d{i}_shape"])
        w = dense_mat(t, rows, cols, seed)
        x = orc.make_input(cols, T, seed)
        assert sha(w) == bytes(d[f"d{i}_w_sha"]) and sha(x) == bytes(d[f"d{i}_x_sha"]), i
        y = orc.matmul_q8(t, w, rows, cols, x)
        assert np.array_equal(y.view(np.uint32), d[f"d{i}_y"].view(np.uint32)), i


def test_oracle_matmul_row_is_vec_dot():
    """Each output is the vec_dot of its row with the token's int8 blocks (no cross-row mixing,
    [T][rows] layout), and a planted row swap is seen."""
    t, rows, cols, T = orc.T_Q4_1, 40, 512, 3
    w = dense_mat(t, rows, cols, 9)
    x = orc.make_input(cols, T, 9)
    y = orc.matmul_q8(t, w, rows, cols, x)
    rb = orc.row_bytes(t, cols)
    for tt in range(T):
        xq = orc.quantize_q8(x[tt])
        for r in (0, 17, rows - 1):
            assert np.float32(orc.vec_dot_q8(t, w[r * rb:(r + 1) * rb], xq, cols)) == y[tt, r]
    w2 = w.copy()
    w2[:rb], w2[rb:2 * rb] = w[rb:2 * rb], w[:rb]
    assert not np.array_equal(orc.matmul_q8(t, w2, rows, cols, x), y)


@pytest.mark.skipif(orc.ref_library_path() is None, reason="oracle/_ref (the reference build) is not built here")
@pytest.mark.parametrize("t,rows,cols,T", [(orc.T_Q4_0, 96, 4096, 5), (orc.T_Q4_1, 33, 1024, 2),
                                           (orc.T_Q6_K, 20, 2048, 3), (orc.T_F32, 24, 1024, 3),
                                           (orc.T_F32, 7, 4096, 1), (orc.T_Q4_0, 17, 96, 3),
                                           (orc.T_Q4_1, 9, 800, 2), (orc.T_Q6_K, 11, 768, 4),
                                           (orc.T_F32, 5, 4128, 2), (orc.T_Q6_K, 3, 256, 1)])
def test_oracle_matmul_matches_reference_live(t, rows, cols, T):
    R = orc.load_ref()

    class QmsMat(ctypes.Structure):   # src/quant.h:11-16
        _fields_ = [("type", ctypes.c_int), ("rows", ctypes.c_int64), ("cols", ctypes.c_int64),
                    ("row_bytes", ctypes.c_uint64), ("data", ctypes.c_void_p)]

    R.qms_matmul.argtypes = [ctypes.POINTER(QmsMat), ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p]
    w = dense_mat(t, rows, cols, 21)
    x = orc.make_input(cols, T, 22) * np.float32(4.0)
    y = np.empty((T, rows), np.float32)
    m = QmsMat(t, rows, cols, orc.row_bytes(t, cols), w.ctypes.data)
    R.qms_matmul(ctypes.byref(m), x.ctypes.data, T, y.ctypes.data)
    assert np.array_equal(orc.matmul_q8(t, w, rows, cols, x).view(np.uint32), y.view(np.uint32))


def typed_dense(t, rows, cols, seed):
    """GGUF bytes of a [rows][cols] matrix of any loader type (expert_types' draws)."""
    import expert_types as et
    return et.expert_bytes(t, rows, cols, 1, seed)


N_CALLS = [   # (type, rows) per matrix, cols, T, --exact
    ([(orc.T_Q8_0, 40)], 256, 3, False),
    ([(orc.T_F16, 17)], 512, 2, False),
    ([(orc.T_Q4_0, 33), (orc.T_Q8_0, 20), (orc.T_F32, 9)], 1024, 4, False),   # one outsider: all exact
    ([(orc.T_Q4_0, 30), (orc.T_Q6_K, 12)], 2048, 2, True),                    # --exact
    ([(orc.T_Q4_1, 25), (orc.T_F32, 8)], 768, 5, False),                      # all fast
]


@pytest.mark.skipif(orc.ref_library_path() is None, reason="oracle/_ref (the reference build) is not built here")
@pytest.mark.parametrize("specs,cols,T,exact", N_CALLS, ids=[f"c{c[1]}_{'_'.join(str(t) for t, _ in c[0])}{'_x' if c[3] else ''}" for c in N_CALLS])
def test_oracle_matmul_n_matches_reference_live(specs, cols, T, exact):
    """qms_matmul_n's call-level choice (src/quant.c:128-142): the fast loop only when every
    matrix of the call is of a fast type and --exact is off, else matmul_exact for all of them;
    the oracle's matmul_n against the reference's, bit for bit."""
    R = orc.load_ref()

    class QmsMat(ctypes.Structure):   # src/quant.h:11-16
        _fields_ = [("type", ctypes.c_int), ("rows", ctypes.c_int64), ("cols", ctypes.c_int64),
                    ("row_bytes", ctypes.c_uint64), ("data", ctypes.c_void_p)]

    ws = [typed_dense(t, r, cols, 30 + i) for i, (t, r) in enumerate(specs)]
    ms = [QmsMat(t, r, cols, orc.row_bytes(t, cols), w.ctypes.data) for (t, r), w in zip(specs, ws)]
    x = orc.make_input(cols, T, 31) * np.float32(2.0)
    ys = [np.empty((T, r), np.float32) for _, r in specs]
    n = len(specs)
    R.qms_matmul_n.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p]
    pw = (ctypes.c_void_p * n)(*[ctypes.addressof(m) for m in ms])
    py = (ctypes.c_void_p * n)(*[y.ctypes.data for y in ys])
    flag = ctypes.c_int.in_dll(R, "qms_exact_math")
    flag.value = 1 if exact else 0
    try:
        R.qms_matmul_n(pw, n, x.ctypes.data, T, py)
    finally:
        flag.value = 0
    got = orc.matmul_n([(t, w, r, cols) for (t, r), w in zip(specs, ws)], x, exact=exact)
    for y, g in zip(ys, got):
        assert np.array_equal(g.view(np.uint32), y.view(np.uint32))
