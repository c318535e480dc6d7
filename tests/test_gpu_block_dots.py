"""Per-block int32 dots of the production expert kernels (src/kernels.c:87-93, 113-119,
148-167): on the probe layers (tests/probe_layers.py) every gate/up row the device computes is
2^-7 x the int32 dot of its designated block and every down row the down block's int32 dot, so
the kernels' own fp32 rows give one block dot per (slot, row) with no instrumentation. Each is
compared with the oracle's orc_block_dot on the device's own int8 inputs, over every slot and
row, on the paths the default batch sizes take: the one-token kernels (decode), the small-batch
and tile kernels, and the MFMA kernels (prefill)."""
import functools

import numpy as np
import pytest

import oracle as orc
import probe_layers as pl

pytestmark = pytest.mark.gpu

CASES = [
    # name, E, X, K, F, T, gate, up, down, path, zipf
    ("q235b_t1", 4096, 128, 8, 1536, 1, orc.T_Q4_0, orc.T_Q4_0, orc.T_Q4_0, "auto", False),
    ("q235b_t4", 4096, 128, 8, 1536, 4, orc.T_Q4_0, orc.T_Q4_0, orc.T_Q4_0, "auto", False),
    ("q235b_t16", 4096, 128, 8, 1536, 16, orc.T_Q4_0, orc.T_Q4_0, orc.T_Q4_0, "auto", False),
    ("q235b_q6k_t64", 4096, 128, 8, 1536, 64, orc.T_Q4_0, orc.T_Q4_0, orc.T_Q6_K, "auto", False),
    ("q235b_q6k_t64_mfma", 4096, 128, 8, 1536, 64, orc.T_Q4_0, orc.T_Q4_0, orc.T_Q6_K, "mfma", False),
    ("q235b_q41_t1", 4096, 128, 8, 1536, 1, orc.T_Q4_0, orc.T_Q4_0, orc.T_Q4_1, "auto", False),
    ("q235b_q6k_t1", 4096, 128, 8, 1536, 1, orc.T_Q4_0, orc.T_Q4_0, orc.T_Q6_K, "auto", False),
    ("q235b_q6k_t3", 4096, 128, 8, 1536, 3, orc.T_Q4_0, orc.T_Q4_0, orc.T_Q6_K, "auto", False),
    ("tiny_q41_q6k_t40", 256, 16, 4, 256, 40, orc.T_Q4_1, orc.T_Q6_K, orc.T_Q4_1, "auto", False),
    ("q235b_gq41_t16", 4096, 128, 8, 1536, 16, orc.T_Q4_1, orc.T_Q4_1, orc.T_Q4_0, "auto", False),
    ("q235b_gq6k_t16", 4096, 128, 8, 1536, 16, orc.T_Q6_K, orc.T_Q6_K, orc.T_Q4_0, "auto", False),
    ("q235b_gq6k_t1", 4096, 128, 8, 1536, 1, orc.T_Q6_K, orc.T_Q6_K, orc.T_Q4_0, "auto", False),
    ("q235b_gq41_t1", 4096, 128, 8, 1536, 1, orc.T_Q4_1, orc.T_Q4_1, orc.T_Q4_0, "auto", False),
    ("q235b_zipf_t512", 4096, 128, 8, 1536, 512, orc.T_Q4_0, orc.T_Q4_0, orc.T_Q4_0, "auto", True),
]


@pytest.fixture(scope="module")
def q():
    from large_model_amd import qmsg
    return qmsg


@functools.lru_cache(maxsize=None)
def _gateup(E, X, K, F, gt, ut):
    return pl.gateup_probe(E, X, K, F, 21, gate_type=gt, up_type=ut)


@functools.lru_cache(maxsize=None)
def _down(E, X, K, F, dt):
    return pl.down_probe(E, X, K, F, 41, down_type=dt)


def _bits(a):
    return np.ascontiguousarray(a).view(np.uint32)


def _run(q, L, x, path):
    with q.Context(L.E, L.X, L.K, L.F, n_layer=1, max_tokens=x.shape[0]) as ctx:
        ctx.upload(0, L.router, (L.types[0], L.gate), (L.types[1], L.up), (L.types[2], L.down))
        ctx.set_path(q.PATH_MFMA if path == "mfma" else q.PATH_AUTO)
        return ctx.moe_debug(0, x)


@pytest.mark.parametrize("name,E,X,K,F,T,gt,ut,dt,path,zipf", CASES, ids=[c[0] for c in CASES])
def test_kernel_block_dots(q, name, E, X, K, F, T, gt, ut, dt, path, zipf):
    from large_model_amd.workloads import zipf_bias
    col0 = zipf_bias(X, K, T, E) if zipf else None
    print(f"[case] block dots {name} gate/up", flush=True)
    L, bg, bu = _gateup(E, X, K, F, gt, ut)
    L = pl.with_router_col0(L, col0)
    x = pl.probe_input(E, T, 30 + T)
    _, d = _run(q, L, x, path)
    assert np.all(d["xq"]["d"] == np.float32(2.0 ** -7))
    exp = pl.expected_gateup(L, bg, bu, d)
    assert np.array_equal(_bits(d["gu"]), _bits(exp)), "gate/up block dots"
    print(f"[case] block dots {name} down", flush=True)
    L, bd = _down(E, X, K, F, dt)
    L = pl.with_router_col0(L, col0)
    x = pl.probe_input(E, T, 50 + T, fixed_blocks=2)
    _, d = _run(q, L, x, path)
    assert np.all(d["gu"][:, :F] == 128.0) and np.all(d["aq"]["d"] == 8.0)
    exp = pl.expected_down(L, bd, d)
    assert np.array_equal(_bits(d["dn"]), _bits(exp)), "down block dots"
    if T <= 16:
        out_ref = L.moe(x)
        out, _ = _run(q, L, x, path)
        assert np.array_equal(_bits(out), _bits(out_ref)), "layer output"
