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
    return orc.synth_mat(t, rows, cols, seed)


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
    wk = orc.make_input(E, 64, 13)
    import expert_types as et
    wv = et.expert_bytes(orc.T_Q8_0, 8, E, 1, 14)
    path = str(tmp_path / "trunk.gguf")
    gf.write_gguf(path, [("general.architecture", gf.STR, "qwen3moe")],
                  [("blk.0.attn_q.weight", orc.T_Q4_0, [E, R], wq.tobytes()),
                   ("blk.0.attn_norm.weight", orc.T_F32, [E], np.ones(E, np.float32).tobytes()),
                   ("blk.0.attn_k.weight", orc.T_F32, [E, 64], wk.tobytes()),
                   ("blk.0.attn_v.weight", orc.T_Q8_0, [E, 8], wv.tobytes())])
    x = orc.make_input(E, 2, 12)
    with q.Gguf(path) as g, q.Context(256, 16, 4, 128, max_tokens=1) as ctx:
        mid = ctx.gguf_upload_mat(g, "blk.0.attn_q.weight")
        (y,) = ctx.matmul_n([mid], x)
        assert np.array_equal(bits(y), bits(orc.matmul_q8(orc.T_Q4_0, wq, R, E, x)))
        kid = ctx.gguf_upload_mat(g, "blk.0.attn_k.weight")       # F32 rows
        qid = ctx.gguf_upload_mat(g, "blk.0.attn_q.weight")
        yk, yq = ctx.matmul_n([kid, qid], x)                       # F32 and Q4_0 in one call
        assert np.array_equal(bits(yk), bits(orc.matmul_q8(orc.T_F32, wk, 64, E, x)))
        assert np.array_equal(bits(yq), bits(y))
        vid = ctx.gguf_upload_mat(g, "blk.0.attn_v.weight")       # Q8_0: matmul_exact, for the whole call
        yv, yq2 = ctx.matmul_n([vid, qid], x)
        assert np.array_equal(bits(yv), bits(orc.matmul_exact(orc.T_Q8_0, wv, 8, E, x)))
        assert np.array_equal(bits(yq2), bits(orc.matmul_exact(orc.T_Q4_0, wq, R, E, x)))
        with pytest.raises(q.QmsgError) as ei:
            ctx.mat_upload(13, np.zeros(176 * 4, np.uint8), 1, 1024)     # Q5_K: no dense kernel
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
            ctx.mat_synth(orc.T_F32, 4, 80, 1)                                 # cols % 32
        assert ei.value.status == -2
        with pytest.raises(q.QmsgError) as ei:
            ctx.mat_synth(orc.T_Q6_K, 4, 640, 1)                               # Q6_K: cols % 256
        assert ei.value.status == -2
        with pytest.raises(q.QmsgError, match="109216") as ei:
            ctx.mat_synth(orc.T_Q4_1, 4, 109248, 1)                            # direct-read kernel's bound
        assert ei.value.status == -2
        with pytest.raises(q.QmsgError, match="2\\^30") as ei:
            ctx.mat_synth(orc.T_Q4_0, 1, 2 ** 31, 1)                           # cols beyond 2^30
        assert ei.value.status == -2


@pytest.mark.parametrize("T", [1, 2, 3, 4, 5, 9])
def test_dense_q6k_and_f32_trunk_shapes(q, T):
    """Q6_K and F32 rows (the other types of qms_matmul's fast path, src/quant.c:128-170): the
    235B trunk's q/k/v shapes in Q6_K (super-blocks staged in chunks of eight), an F32 matrix
    in the same call as a Q4_0 one, and an output-weight-like Q6_K matrix with a ragged row
    count; device-generated matrices checked against the same generator on the host."""
    E, H = 4096, 8192
    print(f"[case] dense q6k/f32 T={T}", flush=True)
    x = orc.make_input(E, T, 20 + T) * np.float32(3.0)
    with q.Context(256, 16, 4, 128, max_tokens=1) as ctx:
        specs = [(orc.T_Q6_K, H, E, 1), (orc.T_Q6_K, 512, E, 2), (orc.T_F32, 512, E, 3), (orc.T_Q4_0, 512, E, 4),
                 (orc.T_Q6_K, 1000, E, 5), (orc.T_F32, 129, E, 6)]
        ids = [ctx.mat_synth(t, r, c, s) for t, r, c, s in specs]
        ys = ctx.matmul_n(ids, x)
    for (t, r, c, s), y in zip(specs, ys):
        ref = orc.matmul_q8(t, dense_mat(t, r, c, s), r, c, x)
        assert np.array_equal(bits(y), bits(ref)), (t, r)


@pytest.mark.parametrize("T", [1, 2, 3, 5, 9, 20])
def test_dense_odd_widths(q, T):
    """Widths the reference's fast path admits (src/quant.c:134-136) off the chunked kernels'
    grid, on the direct-read kernel: F32 / Q4_0 / Q4_1 rows of 96, 800 and 4128 columns (not
    multiples of 256), Q6_K rows of 256, 768 and 4352 (not multiples of 2048) beside Q4 and F32
    rows of the same width on the chunked kernels, ragged row counts, four types in a call."""
    for C in (96, 256, 768, 800, 4128, 4352):
        print(f"[case] dense odd width C={C} T={T}", flush=True)
        x = orc.make_input(C, T, 60 + C) * np.float32(2.0)
        types = [orc.T_Q4_0, orc.T_Q4_1, orc.T_F32] + ([orc.T_Q6_K] if C % 256 == 0 else [])
        specs = [(t, 33 + 17 * i, 70 + i) for i, t in enumerate(types)]
        with q.Context(256, 16, 4, 128, max_tokens=1) as ctx:
            ids = [ctx.mat_synth(t, r, C, s) for t, r, s in specs]
            ys = ctx.matmul_n(ids, x)
        for (t, r, s), y in zip(specs, ys):
            assert np.array_equal(bits(y), bits(orc.matmul_q8(t, dense_mat(t, r, C, s), r, C, x))), (C, t)


def test_dense_direct_read_widest(q):
    """The widest row the direct-read kernel takes (109,216 columns: one token's 3,413 int8
    blocks fill 160 KiB of LDS), Q4_0 and Q4_1, two tokens in two passes."""
    C, T = 109216, 2
    print(f"[case] dense direct-read widest C={C}", flush=True)
    x = orc.make_input(C, T, 61)
    specs = [(orc.T_Q4_0, 7, 81), (orc.T_Q4_1, 5, 82)]
    with q.Context(256, 16, 4, 128, max_tokens=1) as ctx:
        ids = [ctx.mat_synth(t, r, C, s) for t, r, s in specs]
        ys = ctx.matmul_n(ids, x)
    for (t, r, s), y in zip(specs, ys):
        assert np.array_equal(bits(y), bits(orc.matmul_q8(t, dense_mat(t, r, C, s), r, C, x))), t


@pytest.mark.parametrize("T", [1, 3, 6])
def test_dense_f32_wide_rows(q, T):
    """F32 rows of 8192 (attn_output's width: the many-chunk router path) and of 2048."""
    print(f"[case] dense f32 wide T={T}", flush=True)
    with q.Context(256, 16, 4, 128, max_tokens=1) as ctx:
        for C, R in ((8192, 300), (2048, 77)):
            x = orc.make_input(C, T, 40 + C)
            mid = ctx.mat_synth(orc.T_F32, R, C, 9)
            (y,) = ctx.matmul_n([mid], x)
            assert np.array_equal(bits(y), bits(orc.matmul_q8(orc.T_F32, dense_mat(orc.T_F32, R, C, 9), R, C, x))), C


def test_dense_many_tokens_every_type(q):
    """37 tokens: three 16-token passes of the batch kernel (with the separate input
    quantisation) for Q4_0, Q4_1 and Q6_K, three 16-token groups for F32; and T = 0."""
    C, T = 4096, 37
    print(f"[case] dense all types T={T}", flush=True)
    x = orc.make_input(C, T, 50) * np.float32(2.0)
    specs = [(orc.T_Q4_0, 300, 1), (orc.T_Q4_1, 129, 2), (orc.T_Q6_K, 200, 3), (orc.T_F32, 70, 4)]
    with q.Context(256, 16, 4, 128, max_tokens=1) as ctx:
        ids = [ctx.mat_synth(t, r, C, s) for t, r, s in specs]
        ys = ctx.matmul_n(ids, x)
        assert all(y.shape == (0, r) for y, (_, r, _) in zip(ctx.matmul_n(ids, x[:0]), specs))
    for (t, r, s), y in zip(specs, ys):
        assert np.array_equal(bits(y), bits(orc.matmul_q8(t, dense_mat(t, r, C, s), r, C, x))), t


DENSE_TYPES = (orc.T_F32, orc.T_Q4_0, orc.T_Q4_1, orc.T_Q6_K)


@pytest.mark.parametrize("seed", range(40))
def test_dense_random_calls(q, seed):
    """Seeded random calls: one to five matrices of random types (F32, Q4_0, Q4_1, and Q6_K
    where the width is a multiple of 256) and row counts sharing a width of 96-8192 columns,
    1-40 tokens; every product bit for bit against the oracle's qms_matmul."""
    rng = np.random.default_rng(7000 + seed)
    C = int(rng.choice([96, 256, 512, 768, 800, 1024, 2048, 4096, 4128, 4352, 6144, 8192]))
    T = int(rng.choice([1, 1, 2, 3, 4, 5, 8, 16, 17, 40]))
    nm = int(rng.integers(1, 6))
    types = DENSE_TYPES if C % 256 == 0 else DENSE_TYPES[:3]
    specs = [(int(rng.choice(types)), int(rng.integers(1, 1200))) for _ in range(nm)]
    print(f"[case] dense random seed {seed}: C={C} T={T} {specs}", flush=True)
    ws = [dense_mat(t, r, C, 500 + 10 * seed + i) for i, (t, r) in enumerate(specs)]
    x = orc.make_input(C, T, 900 + seed)
    with q.Context(256, 16, 4, 128, max_tokens=1) as ctx:
        ids = [ctx.mat_upload(t, w, r, C) for (t, r), w in zip(specs, ws)]
        ys = ctx.matmul_n(ids, x)
    for (t, r), w, y in zip(specs, ws, ys):
        assert np.array_equal(bits(y), bits(orc.matmul_q8(t, w, r, C, x))), (t, r)


EXACT_CALLS = [   # (type, rows) per matrix, cols, T, the context on QMSG_PATH_FP32
    ([(orc.T_Q8_0, 100)], 2048, 1, False),
    ([(orc.T_F16, 77)], 4096, 3, False),
    ([(orc.T_Q4_0, 300), (orc.T_Q8_0, 64), (orc.T_F32, 40), (orc.T_Q6_K, 33)], 2048, 5, False),
    ([(orc.T_Q4_0, 130), (orc.T_Q6_K, 20), (orc.T_F32, 9)], 4096, 2, True),
    ([(orc.T_Q8_0, 50), (orc.T_F16, 3)], 96, 9, False),
    ([(orc.T_Q4_1, 64)], 8192, 1, True),
]


@pytest.mark.parametrize("specs,cols,T,fp32", EXACT_CALLS,
                         ids=[f"c{c[1]}_t{c[2]}_{'_'.join(str(t) for t, _ in c[0])}{'_fp32' if c[3] else ''}"
                              for c in EXACT_CALLS])
def test_dense_exact_calls(q, specs, cols, T, fp32):
    """qms_matmul_n's matmul_exact (src/quant.c:97-115, 131-141): F16 and Q8_0 matrices, every
    matrix of a call holding one of them, and every call of a context on the --exact path, in
    fp32 chains on dequantised rows; bit for bit against the oracle's matmul_n."""
    import expert_types as et
    print(f"[case] dense exact {specs} C={cols} T={T} fp32={fp32}", flush=True)
    ws = [et.expert_bytes(t, r, cols, 1, 600 + i) for i, (t, r) in enumerate(specs)]
    x = orc.make_input(cols, T, 601) * np.float32(2.0)
    with q.Context(256, 16, 4, 128, max_tokens=1) as ctx:
        if fp32:
            ctx.set_path(q.PATH_FP32)
        ids = [ctx.mat_upload(t, w, r, cols) for (t, r), w in zip(specs, ws)]
        ys = ctx.matmul_n(ids, x)
    ref = orc.matmul_n([(t, w, r, cols) for (t, r), w in zip(specs, ws)], x, exact=fp32)
    for y, r in zip(ys, ref):
        assert np.array_equal(bits(y), bits(r))
