"""The reference's --exact mode on the GPU (QMSG_PATH_FP32): fp32 dequantised rows in one FMA
chain per row, fp32 activations. Output hashed against the reference's own moe() run with
qms_exact_math = 1 (tests/golden/layer_*exact*.npz), and every intermediate against the
oracle, with Q4_0, Q4_1 and Q6_K in every tensor, and switching between the paths."""
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


def bits(a):
    return np.ascontiguousarray(a).view(np.uint32)


@pytest.mark.parametrize("name", ["tiny_exact_t3", "q30b_exact_t2", "q235b_q6k_exact_t1"])
def test_fp32_path_equals_reference_exact_mode(q, name):
    d = dict(np.load(os.path.join(GOLD, f"layer_{name}.npz")))
    E, X, K, F, T, seed, dt, rms = (int(v) for v in d["shape"])
    print(f"[case] fp32 golden {name} T={T}", flush=True)
    x = orc.make_input(E, T, seed, rmsnorm=bool(rms))
    with q.Context(E, X, K, F, n_layer=1, max_tokens=T) as ctx:
        ctx.set_path(q.PATH_FP32)
        ctx.synth(0, seed, down_type=dt)
        out = ctx.moe(0, x)
    assert sha(out) == bytes(d["out_sha"])


CASES = [
    # name, E, X, K, F, T, seed, gate, up, down
    ("tiny_t1", 256, 16, 4, 128, 1, 40, orc.T_Q4_0, orc.T_Q4_0, orc.T_Q4_0),
    ("q30b_t5_q41", 2048, 128, 8, 768, 5, 41, orc.T_Q4_0, orc.T_Q4_0, orc.T_Q4_1),
    ("mixed_q6k_gate_t3", 1024, 32, 4, 512, 3, 42, orc.T_Q6_K, orc.T_Q4_1, orc.T_Q6_K),
    ("q235b_t2", 4096, 128, 8, 1536, 2, 43, orc.T_Q4_0, orc.T_Q4_0, orc.T_Q4_0),
]


@pytest.mark.parametrize("name,E,X,K,F,T,seed,gt,ut,dt", CASES, ids=[c[0] for c in CASES])
def test_fp32_path_intermediates(q, name, E, X, K, F, T, seed, gt, ut, dt):
    print(f"[case] fp32 {name}", flush=True)
    x = orc.make_input(E, T, seed)
    host = orc.Layer(E, X, K, F, seed, gate_type=gt, up_type=ut, down_type=dt, experts=[])
    ref_out, ref = host.moe(x, debug=True, exact=True)
    with q.Context(E, X, K, F, n_layer=1, max_tokens=T) as ctx:
        ctx.synth(0, seed, gate_type=gt, up_type=ut, down_type=dt)
        fast = ctx.moe(0, x)                            # the default (integer) path on the same layer
        ctx.set_path(q.PATH_FP32)
        out, got = ctx.moe_debug(0, x)
        ctx.set_path(q.PATH_AUTO)
        fast_again = ctx.moe(0, x)
    assert np.array_equal(bits(fast), bits(host.moe(x))) and np.array_equal(bits(fast_again), bits(fast))
    assert np.array_equal(bits(got["logits"]), bits(ref["logits"])), "router logits"
    assert np.array_equal(got["sel"], ref["sel"]) and np.array_equal(bits(got["wt"]), bits(ref["wt"]))
    for k in ("start", "slot_t", "slot_of", "active"):
        assert np.array_equal(got[k], ref[k]), k
    assert np.array_equal(bits(got["gu"]), bits(ref["gu"])), "gate/up rows"
    assert np.array_equal(bits(got["act"]), bits(ref["act"])), "activations"
    assert np.array_equal(bits(got["dn"]), bits(ref["dn"])), "down rows"
    assert np.array_equal(bits(out), bits(ref_out)), "layer output"
