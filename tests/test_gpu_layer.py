"""Layer parity on the GPU: libqmsg (HIP, gfx950) against the CPU oracle on identical seeded inputs.

The exact path must reproduce every intermediate bit for bit: router logits, expert ids and
weights, dispatch, the int8 input blocks (xq), gate/up rows, SwiGLU activations, the int8
activation blocks (aq), per-slot down rows and the layer output.
"""
import numpy as np
import pytest

import oracle as orc

pytestmark = pytest.mark.gpu

CASES = [
    # name, E, X, K, F, T, seed, down_type, rmsnorm
    ("tiny_t1", 256, 16, 4, 128, 1, 0, orc.T_Q4_0, False),
    ("tiny_t7", 256, 16, 4, 128, 7, 0, orc.T_Q4_0, False),
    ("q30b_t1", 2048, 128, 8, 768, 1, 1, orc.T_Q4_0, True),
    ("q235b_t1", 4096, 128, 8, 1536, 1, 2, orc.T_Q4_0, False),
    ("q235b_t4", 4096, 128, 8, 1536, 4, 2, orc.T_Q4_0, False),
    ("q235b_t16", 4096, 128, 8, 1536, 16, 2, orc.T_Q4_0, False),
    ("q235b_t8", 4096, 128, 8, 1536, 8, 32, orc.T_Q4_0, False),     # 64 slots: the default path's MFMA down
    ("e768_t9", 768, 32, 4, 256, 9, 33, orc.T_Q4_0, False),         # combine: three 64-thread blocks per token
    ("q30b_q6k_t5", 2048, 128, 8, 768, 5, 3, orc.T_Q6_K, False),
    ("q235b_q6k_t3", 4096, 128, 8, 1536, 3, 4, orc.T_Q6_K, False),
    ("q235b_q6k_t2", 4096, 128, 8, 1536, 2, 31, orc.T_Q6_K, True),   # small-batch down kernel, Q6_K rows
    ("tiny_q41_t3", 256, 16, 4, 128, 3, 9, orc.T_Q4_1, False),
    ("q30b_q41_t1", 2048, 128, 8, 768, 1, 8, orc.T_Q4_1, True),
    ("q235b_q41_t1", 4096, 128, 8, 1536, 1, 7, orc.T_Q4_1, False),
    ("q235b_q41_t6", 4096, 128, 8, 1536, 6, 7, orc.T_Q4_1, False),
    ("q480b_t1", 6144, 160, 8, 2560, 1, 14, orc.T_Q4_0, True),
    ("q480b_q41_t1", 6144, 160, 8, 2560, 1, 15, orc.T_Q4_1, False),
    ("q480b_t5", 6144, 160, 8, 2560, 5, 16, orc.T_Q4_0, False),
    # limits and shapes off the common path
    ("k16_t1", 512, 64, 16, 256, 1, 21, orc.T_Q4_0, False),      # n_used > 8: routed by select
    ("k64_all_t2", 256, 64, 64, 128, 2, 22, orc.T_Q4_0, False),  # every expert used (QMS_MAX_USED)
    ("x256_t3", 256, 256, 8, 128, 3, 23, orc.T_Q4_0, False),     # 256 experts (kernel maximum)
    ("f64_t3", 256, 16, 4, 64, 3, 24, orc.T_Q4_1, False),        # smallest n_ff_exp
    ("q6k_f768_t1", 2048, 128, 8, 768, 1, 25, orc.T_Q6_K, True),  # odd super-blocks per row
    ("q235b_q6k_t1", 4096, 128, 8, 1536, 1, 29, orc.T_Q6_K, False),  # one-token down kernel, Q6_K rows
    ("q480b_q6k_t1", 6144, 160, 8, 2560, 1, 30, orc.T_Q6_K, True),
    # two to four tokens: the small-batch down kernel (several experts per wave, fused combine)
    ("q235b_q41_t3", 4096, 128, 8, 1536, 3, 26, orc.T_Q4_1, False),
    ("q30b_t2", 2048, 128, 8, 768, 2, 27, orc.T_Q4_0, True),
    ("k16_f256_t2", 512, 64, 16, 256, 2, 28, orc.T_Q4_0, False),  # one chunk per row: no cross-expert prefetch
]


def _bits(a):
    return np.ascontiguousarray(a).view(np.uint8)


@pytest.fixture(scope="module")
def qmsg():
    from large_model_amd import qmsg as q
    return q


@pytest.mark.parametrize("name,E,X,K,F,T,seed,dt,rms", CASES, ids=[c[0] for c in CASES])
def test_layer_exact(qmsg, name, E, X, K, F, T, seed, dt, rms):
    print(f"[case] {name} E={E} X={X} K={K} F={F} T={T} seed={seed} down={dt}", flush=True)
    x = orc.make_input(E, T, seed, rmsnorm=rms)
    host = orc.Layer(E, X, K, F, seed, down_type=dt, experts=[])
    ref_out, ref = host.moe(x, debug=True)
    with qmsg.Context(E, X, K, F, n_layer=1, max_tokens=max(T, 1)) as ctx:
        ctx.synth(0, seed, down_type=dt)
        # the device generator wrote the same bytes as the host generator for the used experts
        r, g, u, d = ctx.download(0)
        assert np.array_equal(r, host.router)
        for e in ref["active"]:
            for dev, hst, eb in ((g, host.gate, host.eb[0]), (u, host.up, host.eb[1]), (d, host.down, host.eb[2])):
                assert np.array_equal(dev[e * eb:(e + 1) * eb], hst[e * eb:(e + 1) * eb]), f"expert {e} bytes"
        out, got = ctx.moe_debug(0, x)
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


GATE_UP_CASES = [
    # name, E, X, K, F, T, seed, gate_type, up_type, down_type, rmsnorm
    ("gq41_t1", 2048, 128, 8, 768, 1, 51, orc.T_Q4_1, orc.T_Q4_1, orc.T_Q4_0, True),
    ("gq6k_t4", 4096, 128, 8, 1536, 4, 52, orc.T_Q6_K, orc.T_Q6_K, orc.T_Q6_K, False),
    ("gq6k_uq41_t7", 256, 16, 4, 128, 7, 53, orc.T_Q6_K, orc.T_Q4_1, orc.T_Q4_1, False),
    ("gq40_uq6k_t2", 2048, 128, 8, 768, 2, 54, orc.T_Q4_0, orc.T_Q6_K, orc.T_Q4_0, False),
    ("q480b_gq6k_t3", 6144, 160, 8, 2560, 3, 55, orc.T_Q6_K, orc.T_Q6_K, orc.T_Q4_0, False),
    ("k16_gq41_t1", 512, 64, 16, 256, 1, 56, orc.T_Q4_1, orc.T_Q4_1, orc.T_Q4_0, False),
    ("tiny_gq41_t200", 256, 16, 4, 256, 200, 57, orc.T_Q4_1, orc.T_Q4_1, orc.T_Q6_K, False),
    ("gq6k_t1", 4096, 128, 8, 1536, 1, 58, orc.T_Q6_K, orc.T_Q6_K, orc.T_Q4_0, False),   # streaming Q6_K gate/up
    ("q30b_gq6k_t1", 2048, 128, 8, 768, 1, 59, orc.T_Q6_K, orc.T_Q6_K, orc.T_Q6_K, True),
    ("gq41_t2", 4096, 128, 8, 1536, 2, 60, orc.T_Q4_1, orc.T_Q4_1, orc.T_Q4_1, False),   # streaming Q4_1, two tokens
]


@pytest.mark.parametrize("name,E,X,K,F,T,seed,gt,ut,dt,rms", GATE_UP_CASES, ids=[c[0] for c in GATE_UP_CASES])
def test_layer_gate_up_types(qmsg, name, E, X, K, F, T, seed, gt, ut, dt, rms):
    """Gate and up rows of Q4_1 / Q6_K (and mixed with Q4_0), which the reference's fast path
    takes as well (src/kernels.c:197-200): every intermediate bit for bit, on the default and
    the MFMA path (which hands such layers to the same kernels)."""
    print(f"[case] {name} E={E} X={X} K={K} F={F} T={T} types={gt},{ut},{dt}", flush=True)
    x = orc.make_input(E, T, seed, rmsnorm=rms)
    host = orc.Layer(E, X, K, F, seed, gate_type=gt, up_type=ut, down_type=dt, experts=[])
    ref_out, ref = host.moe(x, debug=True)
    with qmsg.Context(E, X, K, F, n_layer=1, max_tokens=T) as ctx:
        ctx.synth(0, seed, gate_type=gt, up_type=ut, down_type=dt)
        out, got = ctx.moe_debug(0, x)
        ctx.set_path(qmsg.PATH_MFMA)
        out_mfma = ctx.moe(0, x)
    for k in ("sel", "start", "slot_t", "slot_of", "active"):
        assert np.array_equal(got[k], ref[k]), k
    for k in ("logits", "wt", "xq", "gu", "act", "aq", "dn"):
        assert np.array_equal(_bits(got[k]), _bits(ref[k])), k
    assert np.array_equal(_bits(out), _bits(ref_out)), "layer output"
    assert np.array_equal(_bits(out_mfma), _bits(ref_out)), "layer output (MFMA path)"


@pytest.mark.parametrize("scale", [0.0, 1e-38, 1e-30, 300.0])
def test_one_token_routing_ties(qmsg, scale):
    """One-token batches route inside the gate/up kernel. Inputs scaled so every logit is 0,
    or so small that exp(l - max) rounds to the same double for different logits (the exact
    ranking of p then decides, lower index first), or large: selection and weights bit for
    bit against the oracle."""
    E, X, K, F, seed = 2048, 128, 8, 768, 61
    print(f"[case] one-token routing scale={scale}", flush=True)
    x = orc.make_input(E, 1, seed) * np.float32(scale)
    host = orc.Layer(E, X, K, F, seed, experts=[])
    ref_out, ref = host.moe(x, debug=True)
    with qmsg.Context(E, X, K, F, n_layer=1, max_tokens=1) as ctx:
        ctx.synth(0, seed)
        out, got = ctx.moe_debug(0, x)
    assert np.array_equal(got["sel"], ref["sel"]), (got["sel"], ref["sel"])
    assert np.array_equal(_bits(got["wt"]), _bits(ref["wt"])), "routing weights"
    for k in ("start", "slot_t", "slot_of", "active"):
        assert np.array_equal(got[k], ref[k]), k
    # 1e-38: every block's d is below 2^-128, so 1/d is +inf and the codes convert from inf
    assert np.array_equal(_bits(got["xq"]), _bits(ref["xq"])), "int8 input blocks"
    assert np.array_equal(_bits(out), _bits(ref_out)), "layer output"



ONE_TOKEN_CASES = [
    # name, E, X, K, F, seed, down_type, rmsnorm
    ("q235b", 4096, 128, 8, 1536, 71, orc.T_Q4_0, False),
    ("q235b_q41", 4096, 128, 8, 1536, 72, orc.T_Q4_1, True),
    ("q30b", 2048, 128, 8, 768, 73, orc.T_Q4_0, True),
    ("k4_x64", 1024, 64, 4, 512, 74, orc.T_Q4_0, False),
    ("x256", 2048, 256, 8, 256, 75, orc.T_Q4_1, False),
]


@pytest.mark.parametrize("name,E,X,K,F,seed,dt,rms", ONE_TOKEN_CASES, ids=[c[0] for c in ONE_TOKEN_CASES])
def test_one_token_tokens_in_a_row(qmsg, name, E, X, K, F, seed, dt, rms):
    """One-token batches, several tokens in a row on one context (the routing inside the
    gate/up kernel, its published arrays and the down kernel's own quantisation are rewritten
    every call), on the default and the EXACT path: every intermediate bit for bit."""
    print(f"[case] one token {name}", flush=True)
    host = orc.Layer(E, X, K, F, seed, down_type=dt, experts=[])
    with qmsg.Context(E, X, K, F, n_layer=1, max_tokens=1) as ctx:
        ctx.synth(0, seed, down_type=dt)
        for t in range(3):
            x = orc.make_input(E, 1, seed + 100 * t, rmsnorm=rms)
            ref_out, ref = host.moe(x, debug=True)
            for path in (qmsg.PATH_AUTO, qmsg.PATH_EXACT):
                ctx.set_path(path)
                out, got = ctx.moe_debug(0, x)
                for k in ("sel", "start", "slot_t", "slot_of", "active"):
                    assert np.array_equal(got[k], ref[k]), (path, t, k)
                for k in ("logits", "wt", "xq", "gu", "act", "aq", "dn"):
                    assert np.array_equal(_bits(got[k]), _bits(ref[k])), (path, t, k)
                assert np.array_equal(_bits(out), _bits(ref_out)), (path, t, "layer output")


EDGE_CASES = [
    # name, tokens of the case's input, path
    ("nonfinite", (0, 1), "auto"),         # batch: the select kernel
    ("nonfinite", (1,), "auto"),           # one token routed inside the gate/up kernel, every p NaN
    ("nonfinite", (0,), "auto"),           # one token, p = 1 and fifteen p = 0
    ("boundary_underflow", (0,), "auto"),  # logit tie at the top-K boundary, underflowed p
    ("boundary_underflow", (0, 0), "auto"),
    ("nonfinite", (0, 1), "fp32"),         # the --exact mode's routing
]


@pytest.mark.parametrize("name,toks,path", EDGE_CASES, ids=[f"{c[0]}_t{''.join(map(str, c[1]))}_{c[2]}" for c in EDGE_CASES])
def test_routing_edge_cases(qmsg, name, toks, path):
    """A non-finite logit (every p NaN: the reference takes experts 0 .. K-1 with NaN weights)
    and an exact logit tie at the top-K boundary with underflowed p (the lowest untaken index
    wins): expert ids, dispatch and every finite intermediate bit for bit against the oracle,
    NaN weights and outputs in the same places."""
    import routing_cases as rc
    seed = 81 if name == "nonfinite" else 82
    col0, x_all, expect = rc.CASES[name](seed)
    x = np.ascontiguousarray(x_all[list(toks)])
    print(f"[case] routing edge {name} tokens={toks} path={path}", flush=True)
    host = rc.layer(col0, seed)
    exact = path == "fp32"
    ref_out, ref = host.moe(x, debug=True, exact=exact)
    assert np.array_equal(ref["sel"], expect[list(toks)])
    with qmsg.Context(rc.E, rc.X, rc.K, rc.F, n_layer=1, max_tokens=len(toks)) as ctx:
        ctx.synth(0, seed, router_col0=col0)
        if exact:
            ctx.set_path(qmsg.PATH_FP32)
        out, got = ctx.moe_debug(0, x)
    for k in ("sel", "start", "slot_t", "slot_of", "active"):
        assert np.array_equal(got[k], ref[k]), (k, got[k], ref[k])
    assert np.array_equal(_bits(got["logits"]), _bits(ref["logits"])), "router logits"
    assert rc.same_bits_or_both_nan(got["wt"], ref["wt"]), (got["wt"], ref["wt"])
    keys = ("gu", "act", "dn") if exact else ("xq", "gu", "act", "aq", "dn")
    for k in keys:
        assert np.array_equal(_bits(got[k]), _bits(ref[k])), k
    assert rc.same_bits_or_both_nan(out, ref_out), "layer output"
