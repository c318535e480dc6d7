"""Layers at shapes off the integer kernels' grid on the GPU: n_embd % 256 != 0, where the
reference's moe() runs moe_group_exact with the int8 qms_matmul of every slot
(src/model.c:1009-1030, 1090-1093), and n_ff_exp = 32 x odd, where it runs its fast path with
the same numbers. Both take the slot kernels (slot_any_kernel) on every path setting but the
fp32 one, which runs the --exact restatement. Every intermediate bit for bit against the oracle,
whose integer branch is held to the reference build's moe() at such shapes on the CPU
(test_oracle.py::test_off_grid_shapes). With n_embd on the grid and an odd multiple of 32 as
n_ff_exp, gate and up of one streaming type take the integer kernels and only the down rows
the slot kernel."""
import numpy as np
import pytest

import oracle as orc

pytestmark = pytest.mark.gpu

Q40, Q41, Q6K = orc.T_Q4_0, orc.T_Q4_1, orc.T_Q6_K
CASES = [
    # name, E, X, K, F, T, gate, up, down types
    ("e96_f96_t1", 96, 8, 2, 96, 1, Q40, Q40, Q40),
    ("e96_f96_t3", 96, 8, 2, 96, 3, Q40, Q40, Q40),
    ("e288_f160_t5", 288, 12, 3, 160, 5, Q41, Q40, Q41),
    ("e256_f96_t4_q6k", 256, 16, 4, 96, 4, Q6K, Q6K, Q40),
    ("e512_f32_t2", 512, 8, 2, 32, 2, Q40, Q41, Q40),
    ("e800_f256_t1_q6k", 800, 10, 4, 256, 1, Q40, Q40, Q6K),
    ("e2080_f352_t9", 2080, 64, 8, 352, 9, Q40, Q40, Q40),
    ("e4096_f1568_t1", 4096, 32, 8, 1568, 1, Q40, Q40, Q40),
    ("e4096_f1568_t20", 4096, 32, 8, 1568, 20, Q40, Q40, Q41),
    ("e1056_f64_t40", 1056, 32, 4, 64, 40, Q41, Q41, Q41),
    # n_embd on the grid, n_ff_exp an odd multiple of 32, gate and up of one streaming type:
    # the integer routing and gate/up kernels, the slot kernel for the down rows
    ("e2048_f352_t1_hybrid", 2048, 64, 8, 352, 1, Q40, Q40, Q40),
    ("e2048_f352_t5_hybrid", 2048, 64, 8, 352, 5, Q41, Q41, Q40),
    ("e4096_f1568_t24_hybrid", 4096, 32, 8, 1568, 24, Q40, Q40, Q41),
]


def _bits(a):
    return np.ascontiguousarray(a).view(np.uint8)


@pytest.fixture(scope="module")
def q():
    from large_model_amd import qmsg
    return qmsg


@pytest.mark.parametrize("name,E,X,K,F,T,gt,ut,dt", CASES, ids=[c[0] for c in CASES])
def test_off_grid_layer(q, name, E, X, K, F, T, gt, ut, dt):
    print(f"[case] off-grid {name}", flush=True)
    seed = 300 + E % 101 + T
    x = orc.make_input(E, T, seed, rmsnorm=True)
    host = orc.Layer(E, X, K, F, seed, gate_type=gt, up_type=ut, down_type=dt, experts=[])
    ref_out, ref = host.moe(x, debug=True)
    with q.Context(E, X, K, F, n_layer=1, max_tokens=T) as ctx:
        ctx.synth(0, seed, gate_type=gt, up_type=ut, down_type=dt)
        out, got = ctx.moe_debug(0, x)
        for path in (q.PATH_MFMA, q.PATH_EXACT):       # the same slot kernels under every setting
            ctx.set_path(path)
            assert np.array_equal(_bits(ctx.moe(0, x)), _bits(ref_out)), path
    for k in ("sel", "start", "slot_t", "slot_of", "active"):
        assert np.array_equal(got[k], ref[k]), k
    for k in ("logits", "wt", "xq", "gu", "act", "aq", "dn"):
        assert np.array_equal(_bits(got[k]), _bits(ref[k])), k
    assert np.array_equal(_bits(out), _bits(ref_out)), "layer output"


@pytest.mark.parametrize("E,X,K,F,T", [(96, 8, 2, 96, 3), (288, 12, 3, 160, 1), (2080, 64, 8, 352, 6)])
def test_off_grid_fp32_path(q, E, X, K, F, T):
    """The --exact mode at the same kind of shapes (its combine for any n_embd)."""
    print(f"[case] off-grid fp32 E={E} F={F} T={T}", flush=True)
    x = orc.make_input(E, T, 400 + E)
    host = orc.Layer(E, X, K, F, 401, experts=[])
    ref_out = host.moe(x, exact=True)
    with q.Context(E, X, K, F, n_layer=1, max_tokens=T) as ctx:
        ctx.synth(0, 401)
        ctx.set_path(q.PATH_FP32)
        out = ctx.moe(0, x)
    assert np.array_equal(_bits(out), _bits(ref_out))


@pytest.mark.parametrize("E,F,T", [(288, 160, 1), (288, 160, 4), (512, 96, 1)])
def test_off_grid_chain(q, E, F, T):
    """h += moe(l, rmsnorm(h, ffn_norm)) over three layers at n_embd 288 / n_ff_exp 160 and at
    512 / 96, each with the separate rmsnorm launch (the router's fused one runs on the integer
    kernels only, although 512-float rows would fit it)."""
    X, K, NL = 12, 3, 3
    print(f"[case] off-grid chain E={E} F={F} T={T}", flush=True)
    rng = np.random.default_rng(12)
    h0 = orc.make_input(E, T, 79) * np.float32(3.0)
    weights = [rng.uniform(0.5, 1.5, E).astype(np.float32) for _ in range(NL)]
    h = h0.copy()
    for l in range(NL):
        layer = orc.Layer(E, X, K, F, 500 + l, layer=l, down_type=Q41, experts=[])
        h = h + layer.moe(orc.rmsnorm(h, weights[l]))
    with q.Context(E, X, K, F, n_layer=NL, max_tokens=T) as ctx:
        for l in range(NL):
            ctx.synth(l, 500 + l, down_type=Q41)
            ctx.layer_norm(l, weights[l])
        d_h = ctx.device_alloc(h0.nbytes)
        ctx.h2d(d_h, h0)
        ctx.moe_chain(0, NL, d_h, T)
        ctx.sync()
        got = ctx.d2h(d_h, (T, E))
    assert np.array_equal(got.view(np.uint32), h.view(np.uint32))
