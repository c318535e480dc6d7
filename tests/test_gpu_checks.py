"""GPU checks beyond the layer cases: the reference's fixtures hashed directly against the
device output, edge cases uploaded from the host, exact block dots, SiLU/expf bits, the
generator, argument handling and repeated calls."""
import ctypes
import glob
import hashlib
import os

import numpy as np
import pytest

import oracle as orc

pytestmark = pytest.mark.gpu
GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


@pytest.fixture(scope="module")
def q():
    from large_model_amd import qmsg
    return qmsg


def sha(a) -> bytes:
    return hashlib.sha256(np.ascontiguousarray(a).view(np.uint8).tobytes()).digest()


def golden_input(d):
    E, X, K, F, T, seed, dt, rms = (int(v) for v in d["shape"])
    special = str(d["special"])
    x = orc.make_input(E, T, seed, rmsnorm=bool(rms), bias_col0=special == "zipf")
    if special == "zero":
        x[1] = 0.0
    elif special == "large":
        x *= 300.0
    return x


DEVICE_GOLD = ["tiny_t1", "tiny_t7", "q30b_t1", "q235b_t1", "q235b_t4", "q235b_t16", "q235b_q6k_t64",
               "q235b_zipf_t512", "q235b_q41_t1", "q235b_q41_t5", "q480b_t1", "q480b_t2",
               "q30b_gq41_t1", "q235b_gq6k_t4", "tiny_gq6k_uq41_t7"]


@pytest.mark.parametrize("path", ["exact", "auto"])
@pytest.mark.parametrize("name", DEVICE_GOLD)
def test_device_layer_equals_reference_output(q, name, path):
    """Weights generated on the device, output hashed against the reference moe()'s output, on
    the row kernels (exact) and on the default path, which takes the MFMA kernels for the
    16-, 64- and 512-token layers."""
    d = dict(np.load(os.path.join(GOLD, f"layer_{name}.npz")))
    E, X, K, F, T, seed, dt, rms = (int(v) for v in d["shape"])
    print(f"[case] golden {name} T={T} path={path}", flush=True)
    x = golden_input(d)
    col0 = d.get("router_col0")
    gt, ut = (int(v) for v in d.get("gu_types", (q.QMSG_T_Q4_0, q.QMSG_T_Q4_0)))
    with q.Context(E, X, K, F, n_layer=1, max_tokens=T) as ctx:
        ctx.set_path(q.PATH_EXACT if path == "exact" else q.PATH_AUTO)
        ctx.synth(0, seed, gate_type=gt, up_type=ut, down_type=dt, router_col0=col0)
        out = ctx.moe(0, x)
    assert sha(out) == bytes(d["out_sha"])


@pytest.mark.parametrize("name", ["tiny_ties", "tiny_zero_row", "tiny_large"])
def test_uploaded_edge_layers(q, name):
    """Router rows duplicated (exact logit ties), an all-zero input row, large inputs: the
    layer bytes are built on the host and uploaded through qmsg_layer_upload."""
    d = dict(np.load(os.path.join(GOLD, f"layer_{name}.npz")))
    E, X, K, F, T, seed, dt, rms = (int(v) for v in d["shape"])
    L = orc.Layer(E, X, K, F, seed, down_type=dt)
    if str(d["special"]) == "ties":
        L.router[5] = L.router[2]
        L.router[9] = L.router[2]
    x = golden_input(d)
    with q.Context(E, X, K, F, n_layer=1, max_tokens=T) as ctx:
        ctx.upload(0, L.router, (orc.T_Q4_0, L.gate), (orc.T_Q4_0, L.up), (dt, L.down))
        out, dbg = ctx.moe_debug(0, x)
    assert sha(out) == bytes(d["out_sha"])
    _, sel, wt = L.route(x)
    assert np.array_equal(dbg["sel"], sel) and np.array_equal(dbg["wt"].view(np.uint32), wt.view(np.uint32))


def test_block_dots_exact(q):
    """Per-block int32 dots of the device kernels against the oracle's block_dot (Q4_0 gate
    and up, Q6_K and Q4_1 down), random rows/blocks and int8 blocks of widely varying scale."""
    E, X, K, F = 2048, 16, 4, 768
    rng = np.random.default_rng(1)
    with q.Context(E, X, K, F, n_layer=2) as ctx:
        ctx.synth(0, 21, down_type=q.QMSG_T_Q6_K)
        ctx.synth(1, 22, down_type=q.QMSG_T_Q4_1)
        _, g, u, dn = ctx.download(0)
        dn41 = ctx.download(1)[3]
        for layer, which, buf, t, rows, n in ((0, 0, g, orc.T_Q4_0, F, E), (0, 1, u, orc.T_Q4_0, F, E),
                                              (0, 2, dn, orc.T_Q6_K, E, F), (1, 2, dn41, orc.T_Q4_1, E, F)):
            m = 384
            ex = rng.integers(0, X, m).astype(np.int32)
            row = rng.integers(0, rows, m).astype(np.int32)
            blk = rng.integers(0, n // 32, m).astype(np.int32)
            x = rng.standard_normal((m, 32)).astype(np.float32) * rng.uniform(0.01, 50, (m, 1)).astype(np.float32)
            xq = np.concatenate([orc.quantize_q8(x[i]) for i in range(m)])
            print(f"[case] block_dots layer={layer} which={which} m={m}", flush=True)
            got = ctx.block_dots(layer, which, ex, row, blk, xq)
            rb = orc.row_bytes(t, n)
            ref = np.empty(m, np.int32)
            xfull = np.zeros(n // 32, orc.Q8_DTYPE)
            for i in range(m):
                off = (int(ex[i]) * rows + int(row[i])) * rb
                xfull[blk[i]] = xq[i]
                ref[i] = orc.block_dot(t, buf[off:off + rb], xfull, int(blk[i]))
            assert np.array_equal(got, ref), (layer, which)


def test_silu_matches_glibc(q):
    """The device expf restates the C library's expf: SiLU bits must equal a/(1+expf(-a))
    with the C library's expf, over normal, uniform, random-bit and edge inputs."""
    libm = ctypes.CDLL("libm.so.6")
    libm.expf.restype = ctypes.c_float
    libm.expf.argtypes = [ctypes.c_float]
    rng = np.random.default_rng(4)
    x = np.concatenate([
        rng.standard_normal(20000).astype(np.float32) * 4,
        rng.uniform(-104, 90, 20000).astype(np.float32),
        rng.integers(0, 1 << 32, 20000, dtype=np.uint64).astype(np.uint32).view(np.float32),
        np.array([0.0, -0.0, 88.0, -88.0, 88.72, -103.9, -104.0, 1e-45, -1e-45, np.inf, -np.inf], np.float32)])
    x = x[~np.isnan(x)]
    with q.Context(256, 16, 4, 128) as ctx:
        got = ctx.eval_silu(x)
    exp_neg = np.array([libm.expf(float(-v)) for v in x], np.float32)
    with np.errstate(all="ignore"):
        ref = x / (np.float32(1.0) + exp_neg)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got.view(np.uint32)[~nan], ref.view(np.uint32)[~nan])


def test_exp_matches_libc(q):
    """The softmax's device exp (double) equals the C library's exp bit for bit."""
    libm = ctypes.CDLL("libm.so.6")
    libm.exp.restype = ctypes.c_double
    libm.exp.argtypes = [ctypes.c_double]
    rng = np.random.default_rng(5)
    a = rng.standard_normal(8192).astype(np.float32) * 3
    b = rng.standard_normal(8192).astype(np.float32) * 3
    x = np.concatenate([
        -np.abs(a.astype(np.float64) - b.astype(np.float64)),
        -rng.uniform(0, 800, 8192),
        rng.integers(0, 1 << 63, 8192, dtype=np.int64).view(np.float64),
        np.array([0.0, -0.0, -1e-300, -700.0, -708.4, -745.1, -746.0, 709.7, 710.0, -np.inf, np.inf])])
    x = x[~np.isnan(x)]
    got = None
    with q.Context(256, 16, 4, 128) as ctx:
        got = ctx.eval_exp(x)
    ref = np.array([libm.exp(float(v)) for v in x], np.float64)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got.view(np.uint64)[~nan], ref.view(np.uint64)[~nan])


@pytest.mark.parametrize("dt", [orc.T_Q6_K, orc.T_Q4_1])
def test_generator_bytes_identical(q, dt):
    E, X, K, F = 512, 16, 4, 256
    with q.Context(E, X, K, F) as ctx:
        ctx.synth(0, 77, down_type=dt)
        r, g, u, d = ctx.download(0)
    L = orc.Layer(E, X, K, F, 77, down_type=dt)
    assert np.array_equal(r, L.router) and np.array_equal(g, L.gate)
    assert np.array_equal(u, L.up) and np.array_equal(d, L.down)


def test_arguments_and_repeated_calls(q):
    E, X, K, F = 256, 16, 4, 128
    with q.Context(E, X, K, F, n_layer=2, max_tokens=4) as ctx:
        with pytest.raises(q.QmsgError) as ei:
            ctx.moe(0, np.zeros((1, E), np.float32))          # no weights yet
        assert ei.value.status == -1
        ctx.synth(0, 3)
        ctx.synth(1, 4)
        assert ctx.moe(0, np.zeros((0, E), np.float32)).shape == (0, E)     # T = 0
        with pytest.raises(q.QmsgError) as ei:
            ctx.moe(0, np.zeros((5, E), np.float32))
        assert ei.value.status == -5
        with pytest.raises(q.QmsgError):
            ctx.moe(2, np.zeros((1, E), np.float32))
        xs = [orc.make_input(E, t, 100 + t) for t in (1, 4, 2, 3, 1)]
        refs = {l: orc.Layer(E, X, K, F, 3 + l, layer=l) for l in (0, 1)}   # the layer index keys the generator
        for i, x in enumerate(xs):
            l = i % 2
            out = ctx.moe(l, x)
            assert np.array_equal(out.view(np.uint32), refs[l].moe(x).view(np.uint32)), i
