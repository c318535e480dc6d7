"""The layer chain on the GPU (qmsg_moe_chain): for each layer h += moe(l, rmsnorm(h, ffn_norm)),
the MoE half of qms_forward's loop (src/model.c:1283-1285), against the oracle run the same way.
Every step is order-exact (rmsnorm's double chain, the layer, float adds), so the whole chain
must match bit for bit. One-token chains with rows of a multiple of 512 floats (up to 4096) form
each layer's rmsnorm inside the router launch, with h alternating between two rows: odd and even
layer counts end in either."""
import numpy as np
import pytest

import oracle as orc

pytestmark = pytest.mark.gpu

CASES = [
    # name, E, X, K, F, T, n_layer, down_type, with norm weights
    ("tiny_q4_l3_t5", 256, 16, 4, 128, 5, 3, orc.T_Q4_0, False),
    ("q30b_q6k_l3_t4", 2048, 128, 8, 768, 4, 3, orc.T_Q6_K, True),
    ("q30b_q4_l2_t1", 2048, 128, 8, 768, 1, 2, orc.T_Q4_0, True),
    ("tiny_q4_l3_t1", 256, 16, 4, 128, 1, 3, orc.T_Q4_0, True),
    ("q235b_q6k_l1_t1", 4096, 128, 8, 1536, 1, 1, orc.T_Q6_K, True),
    ("q235b_q6k_l3_t1", 4096, 128, 8, 1536, 1, 3, orc.T_Q6_K, True),
    ("q30b_q41_l2_t3", 2048, 128, 8, 768, 3, 2, orc.T_Q4_1, True),
    # the 94-layer stack's shape and batch: MFMA gate/up and Q6_K down between rmsnorm and the
    # residual add
    ("q235b_q6k_l2_t64", 4096, 128, 8, 1536, 64, 2, orc.T_Q6_K, True),
]


@pytest.fixture(scope="module")
def q():
    from large_model_amd import qmsg
    return qmsg


@pytest.mark.parametrize("name,E,X,K,F,T,NL,dt,norm", CASES, ids=[c[0] for c in CASES])
def test_chain_exact(q, name, E, X, K, F, T, NL, dt, norm):
    print(f"[case] chain {name}", flush=True)
    rng = np.random.default_rng(11)
    h0 = orc.make_input(E, T, 77) * np.float32(3.0)
    weights = [rng.uniform(0.5, 1.5, E).astype(np.float32) if norm and l != 1 else None for l in range(NL)]
    seeds = [100 + 7 * l for l in range(NL)]
    # oracle
    h = h0.copy()
    for l in range(NL):
        layer = orc.Layer(E, X, K, F, seeds[l], layer=l, down_type=dt, experts=[])
        xn = orc.rmsnorm(h, weights[l])
        h = h + layer.moe(xn)
    # device
    with q.Context(E, X, K, F, n_layer=NL, max_tokens=T) as ctx:
        for l in range(NL):
            ctx.synth(l, seeds[l], down_type=dt)
            ctx.layer_norm(l, weights[l])
        d_h = ctx.device_alloc(h0.nbytes)
        ctx.h2d(d_h, h0)
        ctx.moe_chain(0, NL, d_h, T)
        ctx.sync()
        got = ctx.d2h(d_h, (T, E))
    assert np.array_equal(got.view(np.uint32), h.view(np.uint32))


@pytest.mark.parametrize("walk", [False, True], ids=["bracket", "walk"])
def test_chain_one_token_modes(q, walk):
    """The fused rmsnorm of one-token chains in both sum modes; in the walk mode every layer's
    row forms its sum in order (counted once per layer)."""
    E, X, K, F, NL, T = 2048, 64, 8, 256, 4, 1
    print(f"[case] one-token chain walk={walk}", flush=True)
    h0 = orc.make_input(E, T, 78)
    h = h0.copy()
    for l in range(NL):
        layer = orc.Layer(E, X, K, F, 200 + l, layer=l, experts=[])
        h = h + layer.moe(orc.rmsnorm(h))
    with q.Context(E, X, K, F, n_layer=NL, max_tokens=T) as ctx:
        for l in range(NL):
            ctx.synth(l, 200 + l)
        d_h = ctx.device_alloc(h0.nbytes)
        ctx.h2d(d_h, h0)
        ctx.rmsnorm_mode(walk)
        ctx.moe_chain(0, NL, d_h, T)
        ctx.sync()
        walked = ctx.rmsnorm_mode(False)
        got = ctx.d2h(d_h, (T, E))
    assert np.array_equal(got.view(np.uint32), h.view(np.uint32))
    if walk:
        assert walked == NL
    else:
        assert walked <= NL


def test_chain_arguments(q):
    E, X, K, F = 256, 16, 4, 128
    with q.Context(E, X, K, F, n_layer=2, max_tokens=2) as ctx:
        ctx.synth(0, 1)
        d_h = ctx.device_alloc(2 * E * 4)
        with pytest.raises(q.QmsgError) as ei:
            ctx.moe_chain(0, 3, d_h, 2)
        assert ei.value.status == -5
        with pytest.raises(q.QmsgError):
            ctx.moe_chain(0, 2, d_h, 2)          # layer 1 has no weights
        with pytest.raises(q.QmsgError) as ei:
            ctx.moe_chain(0, 1, d_h, 3)
        assert ei.value.status == -5
        ctx.moe_chain(0, 1, d_h, 0)              # T = 0: nothing to do
