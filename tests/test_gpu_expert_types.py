"""Expert tensors of types outside the integer fast path on the GPU: Q8_0, F16 and F32 (alone or
mixed with Q4_0 / Q4_1 / Q6_K), which the reference's loader takes and its moe() runs through
moe_group_exact (src/model.c:1009-1030, 1090-1093): each slot's qms_matmul takes int8 blocks
for quantised fast-path types, dot_f32 for F32 rows and matmul_exact's fp32 chain for F16 and
Q8_0 rows. The oracle restates that choice and is held to the reference build's moe() on the
same layers (test_oracle.py::test_expert_types). Every intermediate bit for bit, on every path
setting, and the --exact mode."""
import numpy as np
import pytest

import expert_types as et
import oracle as orc

pytestmark = pytest.mark.gpu

Q40, Q41, Q6K, Q80, F16, F32 = orc.T_Q4_0, orc.T_Q4_1, orc.T_Q6_K, orc.T_Q8_0, orc.T_F16, orc.T_F32
CASES = [   # E, X, K, F, T, (gate, up, down)
    (256, 16, 4, 128, 1, (Q80, Q80, Q80)),
    (256, 16, 4, 128, 3, (Q80, Q80, Q80)),
    (256, 16, 4, 128, 1, (F16, F16, F16)),
    (256, 16, 4, 128, 4, (F32, Q40, F32)),
    (512, 8, 2, 256, 5, (Q40, Q80, Q6K)),
    (96, 8, 2, 96, 2, (Q80, Q41, F16)),
    (288, 12, 3, 96, 3, (Q40, F32, Q40)),
    (2048, 64, 8, 768, 1, (Q80, Q80, Q80)),          # the 30B shape with Q8_0 experts
    (2048, 64, 8, 768, 12, (Q80, Q80, Q6K)),
]


def _bits(a):
    return np.ascontiguousarray(a).view(np.uint8)


@pytest.fixture(scope="module")
def q():
    from large_model_amd import qmsg
    return qmsg


@pytest.mark.parametrize("E,X,K,F,T,types", CASES, ids=["_".join(map(str, c[5])) + f"_e{c[0]}_t{c[4]}" for c in CASES])
def test_expert_types_layer(q, E, X, K, F, T, types):
    print(f"[case] expert types {types} E={E} F={F} T={T}", flush=True)
    seed = 140 + E % 83 + T
    L = et.typed_layer(E, X, K, F, types, seed)
    x = orc.make_input(E, T, seed, rmsnorm=True)
    ref_out, ref = L.moe(x, debug=True)
    ref_exact = L.moe(x, exact=True)
    with q.Context(E, X, K, F, n_layer=1, max_tokens=T) as ctx:
        ctx.upload(0, L.router, (types[0], L.gate), (types[1], L.up), (types[2], L.down))
        out, got = ctx.moe_debug(0, x)
        for path in (q.PATH_MFMA, q.PATH_EXACT):
            ctx.set_path(path)
            assert np.array_equal(_bits(ctx.moe(0, x)), _bits(ref_out)), path
        ctx.set_path(q.PATH_FP32)
        assert np.array_equal(_bits(ctx.moe(0, x)), _bits(ref_exact)), "fp32 path"
    for k in ("sel", "start", "slot_t", "slot_of", "active"):
        assert np.array_equal(got[k], ref[k]), k
    for k in ("logits", "wt", "xq", "gu", "act", "aq", "dn"):
        assert np.array_equal(_bits(got[k]), _bits(ref[k])), k
    assert np.array_equal(_bits(out), _bits(ref_out)), "layer output"


def test_expert_types_refusals(q):
    """F32 up with quantised gate and down at n_embd % 256 == 0 (the reference's fast path has
    no F32 dot for it: its output is zero there) is refused at upload, and the device generator
    writes only Q4_0 / Q4_1 / Q6_K."""
    E, X, K, F = 256, 16, 4, 128
    L = et.typed_layer(E, X, K, F, (Q40, F32, Q40), 5)
    with q.Context(E, X, K, F, n_layer=1, max_tokens=1) as ctx:
        with pytest.raises(q.QmsgError) as ei:
            ctx.upload(0, L.router, (Q40, L.gate), (F32, L.up), (Q40, L.down))
        assert ei.value.status == -2
        with pytest.raises(q.QmsgError) as ei:
            ctx.synth(0, 5, gate_type=Q80)
        assert ei.value.status == -2
