"""Dense (trunk) products on the GPU: qmsg_matmul_n against the reference's qms_matmul outputs
(tests/golden/dense.npz) and the oracle, bit for bit, at the 235B trunk's shapes (attn_q/k/v
as one call, attn_output), with row tails, Q4_1 rows, several token counts, device buffers,
a GGUF-loaded matrix and the argument checks."""
import hashlib
import os

import numpy as np
import pytest

import gguf_file as gf
import oracle as orc

pytestmark = pytest.mark.gpu
GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


@pytest.fixture(scope="module")
def q():
    from large_model_amd import qmsg
    return qmsg


def dense_mat(t, rows, cols, seed):
    w = np.zeros(rows * orc.row_bytes(t, cols), np.uint8)
    orc.lib.orc_synth_experts(seed, 0, orc.KIND_GATE, t, rows, cols, 0, 1, 0.02, w.ctypes.data)
    return w


def bits(a):
    return np.ascontiguousarray(a).view(np.uint32)


def test_dense_reference_fixtures(q):
    d = dict(np.load(os.path.join(GOLD, "dense.npz")))
    with q.Context(256, 16, 4, 128, max_tokens=1) as ctx:
        for i in range(int(d["n_dense_cases"])):
            t, rows, cols, T, seed = (int(v) for v in d[f"d{i}_shape"])
            print(f"[case] dense fixture {i}: type={t} {rows}x{cols} T={T}", flush=True)
            w = dense_mat(t, rows, cols, seed)
            x = orc.make_input(cols, T, seed)
            mid = ctx.mat_upload(t, w, rows, cols)
            (y,) = ctx.matmul_n([mid], x)
            assert np.array_equal(bits(y), bits(d[f"d{i}_y"])), i


@pytest.mark.parametrize("T", [1, 2, 5, 16])
def test_dense_qkv_and_output_235b_shapes(q, T):
    """attn_q [8192 x 4096], attn_k / attn_v [512 x 4096] in one qms_matmul_n call, then
    attn_output [4096 x 8192] (Q4_0), as the 235B trunk does per layer (src/model.c:442, 494)."""
    E, H = 4096, 8192
    print(f"[case] dense qkv/o T={T}", flush=True)
    wq, wk, wv = dense_mat(orc.T_Q4_0, H, E, 1), dense_mat(orc.T_Q4_0, 512, E, 2), dense_mat(orc.T_Q4_0, 512, E, 3)
    wo = dense_mat(orc.T_Q4_0, E, H, 4)
    x = orc.make_input(E, T, 5)
    a = orc.make_input(H, T, 6) * np.float32(2.0)
    with q.Context(256, 16, 4, 128, max_tokens=1) as ctx:
        ids = [ctx.mat_upload(orc.T_Q4_0, wq, H, E), ctx.mat_upload(orc.T_Q4_0, wk, 512, E),
               ctx.mat_upload(orc.T_Q4_0, wv, 512, E)]
        io = ctx.mat_upload(orc.T_Q4_0, wo, E, H)
        ys = ctx.matmul_n(ids, x)
        (yo,) = ctx.matmul_n([io], a)
    for y, w, rows in zip(ys, (wq, wk, wv), (H, 512, 512)):
        assert np.array_equal(bits(y), bits(orc.matmul_q8(orc.T_Q4_0, w, rows, E, x)))
    assert np.array_equal(bits(yo), bits(orc.matmul_q8(orc.T_Q4_0, wo, E, H, a)))


@pytest.mark.parametrize("T", [1, 3])
def test_dense_mixed_types_tails_and_device_buffers(q, T):
    """Q4_0 and Q4_1 matrices in one call (two launches), row counts that are not multiples
    of 8 or 16, more than four matrices, and the device-buffer entry point (one token: eight
    lanes per row; three: four)."""
    C = 2048
    shapes = [(orc.T_Q4_1, 1000), (orc.T_Q4_0, 17), (orc.T_Q4_1, 16), (orc.T_Q4_0, 1), (orc.T_Q4_0, 300),
              (orc.T_Q4_1, 65)]
    ws = [dense_mat(t, r, C, 30 + i) for i, (t, r) in enumerate(shapes)]
    x = orc.make_input(C, T, 7) * np.float32(10.0)
    with q.Context(256, 16, 4, 128, max_tokens=1) as ctx:
        ids = [ctx.mat_upload(t, w, r, C) for (t, r), w in zip(shapes, ws)]
        ys = ctx.matmul_n(ids, x)
        d_x = ctx.device_alloc(x.nbytes)
        ctx.h2d(d_x, x)
        d_ys = [ctx.device_alloc(T * r * 4) for _, r in shapes]
        ctx.matmul_n_device(ids, d_x, T, d_ys)
        ctx.sync()
        dev = [ctx.d2h(p, (T, r)) for p, (_, r) in zip(d_ys, shapes)]
    for (t, r), w, y, yd in zip(shapes, ws, ys, dev):
        ref = orc.matmul_q8(t, w, r, C, x)
        assert np.array_equal(bits(y), bits(ref)), (t, r)
        assert np.array_equal(bits(yd), bits(ref)), (t, r)


def test_dense_from_gguf_and_errors(q, tmp_path):
    E, R = 1024, 256
    wq = dense_mat(orc.T_Q4_0, R, E, 11)
    path = str(tmp_path / "trunk.gguf")
    gf.write_gguf(path, [("general.architecture", gf.STR, "qwen3moe")],
                  [("blk.0.attn_q.weight", orc.T_Q4_0, [E, R], wq.tobytes()),
                   ("blk.0.attn_norm.weight", orc.T_F32, [E], np.ones(E, np.float32).tobytes()),
                   ("blk.0.attn_k.weight", orc.T_F32, [E, 64], np.zeros((64, E), np.float32).tobytes())])
    x = orc.make_input(E, 2, 12)
    with q.Gguf(path) as g, q.Context(256, 16, 4, 128, max_tokens=1) as ctx:
        mid = ctx.gguf_upload_mat(g, "blk.0.attn_q.weight")
        (y,) = ctx.matmul_n([mid], x)
        assert np.array_equal(bits(y), bits(orc.matmul_q8(orc.T_Q4_0, wq, R, E, x)))
        with pytest.raises(q.QmsgError) as ei:
            ctx.gguf_upload_mat(g, "blk.0.attn_k.weight")         # F32 rows: not a dense kernel type
        assert ei.value.status == -2
        with pytest.raises(q.QmsgError):
            ctx.gguf_upload_mat(g, "blk.0.attn_norm.weight")      # 1-D
        with pytest.raises(q.QmsgError):
            ctx.gguf_upload_mat(g, "blk.9.attn_q.weight")         # missing
        other = ctx.mat_upload(orc.T_Q4_0, dense_mat(orc.T_Q4_0, 16, 512, 1), 16, 512)
        with pytest.raises(q.QmsgError):
            ctx.matmul_n([mid, other], x)                          # cols differ
        with pytest.raises(q.QmsgError):
            ctx.matmul_n([mid + 5], x)                             # unknown id
        with pytest.raises(q.QmsgError) as ei:
            ctx.mat_upload(orc.T_Q4_0, dense_mat(orc.T_Q4_0, 4, 96, 1), 4, 96)   # cols % 256
        assert ei.value.status == -2
