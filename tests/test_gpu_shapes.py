"""Expert counts and top-k widths away from the 128 / 8 of the benchmark shapes on the GPU: a
Mixtral-like layer (8 experts, top 2, n_ff_exp 14336), a small 8-expert layer, a 60-expert one,
the largest count taken (256: four logits per lane of the one-token routing), 200 experts (a
partly filled last group of 64), top 1, top 16 / 64 (past the one-token and small-batch
kernels' eight selections per token) and top 8 of 8 (no expert past the top-K boundary), each
at one token (routing inside the gate/up kernel), two to four tokens (select, the small-batch
down kernel), a batch on the MFMA kernels, and the fp32 path. Every intermediate bit for bit
against the oracle, as in test_gpu_layer.py; the reference's fast path has no condition on the
expert count (src/model.c:1090-1093)."""
import numpy as np
import pytest

import oracle as orc

pytestmark = pytest.mark.gpu

CASES = [
    # name, E, X, K, F, T, seed, down type, path
    ("x8_k2_t1", 256, 8, 2, 128, 1, 101, orc.T_Q4_0, "auto"),
    ("x8_k2_t3", 256, 8, 2, 128, 3, 102, orc.T_Q4_0, "auto"),
    ("x8_k2_t40_mfma", 256, 8, 2, 256, 40, 103, orc.T_Q4_1, "auto"),
    ("x60_k4_t1", 1024, 60, 4, 256, 1, 104, orc.T_Q4_0, "auto"),
    ("x60_k4_t4", 1024, 60, 4, 256, 4, 105, orc.T_Q6_K, "auto"),
    ("x60_k4_t64", 1024, 60, 4, 256, 64, 106, orc.T_Q4_0, "auto"),
    ("x60_k4_t5_exact", 1024, 60, 4, 256, 5, 107, orc.T_Q4_0, "exact"),
    ("mixtral_t1", 4096, 8, 2, 14336, 1, 108, orc.T_Q4_0, "auto"),
    ("mixtral_t4", 4096, 8, 2, 14336, 4, 109, orc.T_Q4_0, "auto"),
    ("x256_k8_t1", 1024, 256, 8, 256, 1, 121, orc.T_Q4_0, "auto"),
    ("x256_k8_t1_q6k", 1024, 256, 8, 256, 1, 122, orc.T_Q6_K, "auto"),
    ("x256_k8_t4", 1024, 256, 8, 256, 4, 123, orc.T_Q6_K, "auto"),
    ("x256_k8_t48", 1024, 256, 8, 256, 48, 124, orc.T_Q4_0, "auto"),
    ("x200_k6_t1", 1024, 200, 6, 256, 1, 125, orc.T_Q4_1, "auto"),
    ("x200_k6_t3", 1024, 200, 6, 256, 3, 126, orc.T_Q4_0, "auto"),
    ("x64_k1_t1", 512, 64, 1, 128, 1, 127, orc.T_Q4_0, "auto"),
    ("x64_k1_t5", 512, 64, 1, 128, 5, 128, orc.T_Q4_0, "auto"),
    ("x64_k1_t40", 512, 64, 1, 256, 40, 129, orc.T_Q6_K, "auto"),
    ("x256_k16_t1", 1024, 256, 16, 256, 1, 130, orc.T_Q4_0, "auto"),
    ("x256_k16_t2", 1024, 256, 16, 256, 2, 131, orc.T_Q4_0, "auto"),
    ("x256_k64_t1", 1024, 256, 64, 256, 1, 132, orc.T_Q4_0, "auto"),
    ("x256_k64_t3", 1024, 256, 64, 256, 3, 133, orc.T_Q4_1, "auto"),
    ("x8_k8_t1", 256, 8, 8, 128, 1, 134, orc.T_Q4_0, "auto"),      # every expert selected
    ("x8_k8_t2", 256, 8, 8, 128, 2, 135, orc.T_Q4_0, "auto"),
]


def _bits(a):
    return np.ascontiguousarray(a).view(np.uint8)


@pytest.fixture(scope="module")
def q():
    from large_model_amd import qmsg
    return qmsg


@pytest.mark.parametrize("name,E,X,K,F,T,seed,dt,path", CASES, ids=[c[0] for c in CASES])
def test_expert_counts(q, name, E, X, K, F, T, seed, dt, path):
    print(f"[case] shapes {name} E={E} X={X} K={K} F={F} T={T} path={path}", flush=True)
    x = orc.make_input(E, T, seed, rmsnorm=True)
    host = orc.Layer(E, X, K, F, seed, down_type=dt, experts=[])
    ref_out, ref = host.moe(x, debug=True)
    with q.Context(E, X, K, F, n_layer=1, max_tokens=T) as ctx:
        ctx.synth(0, seed, down_type=dt)
        ctx.set_path(q.PATH_EXACT if path == "exact" else q.PATH_AUTO)
        out, got = ctx.moe_debug(0, x)
        out2 = ctx.moe(0, x)
    for k in ("sel", "start", "slot_t", "slot_of", "active"):
        assert np.array_equal(got[k], ref[k]), k
    for k in ("logits", "wt", "xq", "gu", "act", "aq", "dn"):
        assert np.array_equal(_bits(got[k]), _bits(ref[k])), k
    assert np.array_equal(_bits(out), _bits(ref_out)), "layer output"
    assert np.array_equal(_bits(out2), _bits(ref_out)), "second call"


@pytest.mark.parametrize("E,X,K,F,T,seed", [(256, 8, 2, 128, 3, 111), (1024, 60, 4, 256, 2, 112),
                                             (1024, 256, 8, 256, 2, 113), (512, 64, 1, 128, 1, 114)])
def test_expert_counts_fp32_path(q, E, X, K, F, T, seed):
    """The --exact mode at the same expert counts."""
    print(f"[case] shapes fp32 X={X} T={T}", flush=True)
    x = orc.make_input(E, T, seed)
    host = orc.Layer(E, X, K, F, seed, experts=[])
    ref_out = host.moe(x, exact=True)
    with q.Context(E, X, K, F, n_layer=1, max_tokens=T) as ctx:
        ctx.synth(0, seed)
        ctx.set_path(q.PATH_FP32)
        out = ctx.moe(0, x)
    assert np.array_equal(_bits(out), _bits(ref_out))
