"""Seeded random layers on the GPU: n_embd, expert count, n_used, n_ff_exp, batch size, the three
weight types (gate and up mostly alike) and the integer paths (auto, the row kernels only, the
MFMA kernels forced) drawn per case; every intermediate bit for bit against the oracle, as in
test_gpu_layer.py. Half the cases are at the benchmark widths (n_embd 4096 / 6144, n_ff_exp 768
to 2560). 820 cases of the same generator have been run once, with no difference."""
import numpy as np
import pytest

import oracle as orc

pytestmark = pytest.mark.gpu

T4, T41, T6 = orc.T_Q4_0, orc.T_Q4_1, orc.T_Q6_K


def draw(seed: int, big: bool):
    rng = np.random.default_rng(seed)
    E = int(rng.choice([4096, 4096, 6144])) if big else int(rng.choice([256, 512, 768, 1024, 2048]))
    X = int(rng.choice([4, 8, 16, 32, 60, 64, 100, 128, 160, 256]))
    K = int(min(X, rng.choice([1, 2, 4, 6, 8, 8, 8, 12, 16])))
    F = int(rng.choice([1536, 2560, 768])) if big else int(rng.choice([128, 256, 512, 768, 1024]))
    gt = int(rng.choice([T4, T41, T6])) if rng.random() < 0.3 else T4
    ut = gt if rng.random() < 0.8 else int(rng.choice([T4, T41, T6]))
    dt = int(rng.choice([T4, T41, T6]))
    if F % 256 and dt == T6:
        dt = T4
    T = int(rng.choice([1, 1, 2, 3, 4, 5, 8, 12, 16, 24, 33, 40, 64, 96, 128, 200]))
    path = str(rng.choice(["auto", "auto", "auto", "exact", "mfma"]))
    while E * F * T * K > 1.0e9 and T > 1:     # keeps the oracle's share of each case short
        T //= 2
    rms = bool(rng.random() < 0.5)
    return E, X, K, F, T, gt, ut, dt, path, rms


CASES = [(s, False) for s in range(3000, 3030)] + [(s, True) for s in range(6000, 6030)]


def _bits(a):
    return np.ascontiguousarray(a).view(np.uint8)


@pytest.fixture(scope="module")
def q():
    from large_model_amd import qmsg
    return qmsg


@pytest.mark.parametrize("seed,big", CASES, ids=[f"{'big' if b else 'small'}{s}" for s, b in CASES])
def test_random_layer(q, seed, big):
    E, X, K, F, T, gt, ut, dt, path, rms = draw(seed, big)
    print(f"[case] random seed {seed}: E={E} X={X} K={K} F={F} T={T} types={gt},{ut},{dt} path={path}",
          flush=True)
    x = orc.make_input(E, T, seed, rmsnorm=rms)
    host = orc.Layer(E, X, K, F, seed, gate_type=gt, up_type=ut, down_type=dt, experts=[])
    ref_out, ref = host.moe(x, debug=True)
    with q.Context(E, X, K, F, n_layer=1, max_tokens=T) as ctx:
        ctx.synth(0, seed, gate_type=gt, up_type=ut, down_type=dt)
        ctx.set_path({"auto": q.PATH_AUTO, "exact": q.PATH_EXACT, "mfma": q.PATH_MFMA}[path])
        out, got = ctx.moe_debug(0, x)
        out2 = ctx.moe(0, x)
    for k in ("sel", "start", "slot_t", "slot_of", "active"):
        assert np.array_equal(got[k], ref[k]), k
    for k in ("logits", "wt", "xq", "gu", "act", "aq", "dn"):
        assert np.array_equal(_bits(got[k]), _bits(ref[k])), k
    assert np.array_equal(_bits(out), _bits(ref_out)), "layer output"
    assert np.array_equal(_bits(out2), _bits(ref_out)), "second call"
