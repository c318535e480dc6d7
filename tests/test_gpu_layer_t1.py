"""One-token layers on the GPU beyond the shapes of test_gpu_layer.py: every intermediate bit
for bit against the oracle, repeated calls on one context (layers, inputs and batch sizes
alternating, the allocation-free entry among them), and routing cases whose logit order points
at experts the exact selection does not take, so the gate/up kernel's speculative stream must
be replaced by the selected experts' rows."""
import numpy as np
import pytest

import oracle as orc

pytestmark = pytest.mark.gpu

CASES = [
    # name, E, X, K, F, seed, gate/up type, down type, rmsnorm
    ("q235b_q6k", 4096, 128, 8, 1536, 29, orc.T_Q4_0, orc.T_Q6_K, False),
    ("q30b_gq41_q6k", 2048, 128, 8, 768, 61, orc.T_Q4_1, orc.T_Q6_K, True),
    ("k4_e1024", 1024, 32, 4, 512, 62, orc.T_Q4_0, orc.T_Q4_0, False),
    ("x256", 2048, 256, 8, 256, 63, orc.T_Q4_1, orc.T_Q4_1, False),
    ("f2048", 1024, 64, 8, 2048, 64, orc.T_Q4_0, orc.T_Q6_K, False),
]


def _bits(a):
    return np.ascontiguousarray(a).view(np.uint8)


@pytest.fixture(scope="module")
def qmsg():
    from large_model_amd import qmsg as q
    return q


def _check(got, out, ref, ref_out):
    assert np.array_equal(_bits(got["logits"]), _bits(ref["logits"])), "router logits"
    assert np.array_equal(got["sel"], ref["sel"]), "expert ids"
    assert np.array_equal(_bits(got["wt"]), _bits(ref["wt"])), "routing weights"
    for k in ("start", "slot_t", "slot_of", "active"):
        assert np.array_equal(got[k], ref[k]), k
    assert np.array_equal(_bits(got["xq"]), _bits(ref["xq"])), "int8 input blocks"
    assert np.array_equal(_bits(got["gu"]), _bits(ref["gu"])), "gate/up rows"
    assert np.array_equal(_bits(got["act"]), _bits(ref["act"])), "swiglu"
    assert np.array_equal(_bits(got["aq"]), _bits(ref["aq"])), "int8 activation blocks"
    assert np.array_equal(_bits(got["dn"]), _bits(ref["dn"])), "down rows"
    assert np.array_equal(_bits(out), _bits(ref_out)), "layer output"


@pytest.mark.parametrize("name,E,X,K,F,seed,gt,dt,rms", CASES, ids=[c[0] for c in CASES])
def test_one_token_layer(qmsg, name, E, X, K, F, seed, gt, dt, rms):
    print(f"[case] one-token layer {name}", flush=True)
    x = orc.make_input(E, 1, seed, rmsnorm=rms)
    host = orc.Layer(E, X, K, F, seed, gate_type=gt, up_type=gt, down_type=dt, experts=[])
    ref_out, ref = host.moe(x, debug=True)
    with qmsg.Context(E, X, K, F, n_layer=1, max_tokens=2) as ctx:
        ctx.synth(0, seed, gate_type=gt, up_type=gt, down_type=dt)
        out, got = ctx.moe_debug(0, x)
        _check(got, out, ref, ref_out)
        out2 = ctx.moe(0, x)          # again, without the debug copies
        assert np.array_equal(_bits(out2), _bits(ref_out)), "second call"


def test_one_token_calls_in_a_row(qmsg):
    """Layers, inputs and batch sizes alternate on one context, and the allocation-free entry
    (the device's static scratch) takes every other call."""
    E, X, K, F = 2048, 128, 8, 768
    print("[case] one-token calls in a row", flush=True)
    hosts = [orc.Layer(E, X, K, F, 70 + l, layer=l, experts=[]) for l in range(2)]
    with qmsg.Context(E, X, K, F, n_layer=2, max_tokens=3) as ctx:
        for l in range(2):
            ctx.synth(l, 70 + l)
        d_x = ctx.device_alloc(3 * E * 4)
        d_y = ctx.device_alloc(3 * E * 4)
        plan = [(0, 1), (1, 1), (0, 3), (0, 1), (1, 1), (1, 2), (1, 1), (0, 1)]
        for i, (l, T) in enumerate(plan):
            x = orc.make_input(E, T, 500 + i)
            ref = hosts[l].moe(x)
            ctx.h2d(d_x, x)
            if i % 2:
                ctx.moe_device_noalloc(l, d_x, T, d_y)
            else:
                ctx.moe_device(l, d_x, T, d_y)
            ctx.sync()
            got = ctx.d2h(d_y, (T, E))
            assert np.array_equal(_bits(got), _bits(ref)), f"call {i} (layer {l}, T={T})"


def _edge_case(name, E, X, seed):
    """The routing edge cases of routing_cases.py at a width where the one-token down kernel
    runs (n_ff_exp 256)."""
    col0 = orc.synth_f32(seed, 0, orc.KIND_ROUTER, 0, X * E, 0.02).reshape(X, E)[:, 0].copy()
    if name == "nonfinite":
        col0[5] = np.float32(3e38)
        x = orc.make_input(E, 2, seed)
        x[0, 0] = 0.5      # expert 5 leads, every other p underflows to 0
        x[1, 0] = 2.0      # an infinite logit: every p is NaN, experts 0 .. K-1 are taken
        return col0, x
    col0[:] = 0.0
    col0[10], col0[11], col0[12] = 2000.0, 1999.0, 1998.0
    col0[13] = col0[14] = 1000.0
    col0[2] = 500.0
    x = np.zeros((1, E), np.float32)
    x[0, 0] = 1.0          # logits = col0 exactly: the fourth pick is expert 0, not 13
    return col0, x


EDGE = [("nonfinite", 0), ("nonfinite", 1), ("boundary_underflow", 0)]


@pytest.mark.parametrize("name,tok", EDGE, ids=[f"{n}_t{t}" for n, t in EDGE])
def test_one_token_routing_edges(qmsg, name, tok):
    import routing_cases as rc
    E, X, K, F, seed = 1024, 16, 4, 256, 90
    print(f"[case] one-token routing edge {name} token {tok}", flush=True)
    col0, x_all = _edge_case(name, E, X, seed)
    x = np.ascontiguousarray(x_all[tok:tok + 1])
    host = orc.Layer(E, X, K, F, seed, experts=[], router_col0=col0)
    ref_out, ref = host.moe(x, debug=True)
    logit_top = np.argsort(-ref["logits"][0], kind="stable")[:K]
    assert set(logit_top.tolist()) != set(ref["sel"].ravel().tolist()), "the logit order must mislead"
    with qmsg.Context(E, X, K, F, n_layer=1, max_tokens=1) as ctx:
        ctx.synth(0, seed, router_col0=col0)
        out, got = ctx.moe_debug(0, x)
    for k in ("sel", "start", "slot_t", "slot_of", "active"):
        assert np.array_equal(got[k], ref[k]), (k, got[k], ref[k])
    assert np.array_equal(_bits(got["logits"]), _bits(ref["logits"])), "router logits"
    assert rc.same_bits_or_both_nan(got["wt"], ref["wt"]), (got["wt"], ref["wt"])
    for k in ("xq", "gu", "act", "aq", "dn"):
        assert np.array_equal(_bits(got[k]), _bits(ref[k])), k
    assert rc.same_bits_or_both_nan(out, ref_out), "layer output"
