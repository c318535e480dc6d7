"""Seeded random layers on the GPU: n_embd, expert count, n_used, n_ff_exp, batch size, the three
weight types (gate and up mostly alike) and the integer paths (auto, the row kernels only, the
MFMA kernels forced) drawn per case; every intermediate bit for bit against the oracle, as in
test_gpu_layer.py. Half the cases are at the benchmark widths (n_embd 4096 / 6144, n_ff_exp 768
to 2560). 820 cases of the same generator have been run once, with no difference. A second
generator draws layers for the slot kernels (widths off the integer grid, Q8_0 / F16 / F32
expert tensors, every path setting including fp32); 500 of its cases were run once, with no
difference."""
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


Q80, F16, F32 = orc.T_Q8_0, orc.T_F16, orc.T_F32


def draw_slot(seed: int):
    """A layer for the slot kernels: a width off the integer grid, or expert tensors outside
    the integer fast path (Q8_0 / F16 / F32 among Q4_0 / Q4_1 / Q6_K), or both."""
    rng = np.random.default_rng(seed)
    E = int(rng.choice([96, 160, 256, 288, 512, 800, 1056, 2048, 2080]))
    F = int(rng.choice([32, 64, 96, 128, 160, 256, 352, 768]))
    X = int(rng.choice([4, 8, 12, 16, 32, 60, 64, 128]))
    K = int(min(X, rng.choice([1, 2, 3, 4, 6, 8])))
    pool = [T4, T41, Q80, F16, F32] + ([T6] if E % 256 == 0 else [])
    gt, ut = int(rng.choice(pool)), int(rng.choice(pool))
    dpool = [T4, T41, Q80, F16, F32] + ([T6] if F % 256 == 0 else [])
    dt = int(rng.choice(dpool))
    quant = (T4, T41, T6)
    if E % 256 == 0 and F % 64 == 0 and all(t in quant for t in (gt, ut, dt)):
        gt = Q80                                   # off the integer kernels
    if ut == F32 and gt in quant + (F32,) and gt != F32 and dt in quant and E % 256 == 0:
        ut = Q80                                   # the combination the library refuses
    T = int(rng.choice([1, 2, 3, 5, 8, 13, 24]))
    path = str(rng.choice(["auto", "auto", "exact", "mfma", "fp32"]))
    return E, X, K, F, T, (gt, ut, dt), path


SLOT_SEEDS = list(range(8000, 8030))


@pytest.mark.parametrize("seed", SLOT_SEEDS)
def test_random_slot_layer(q, seed):
    import expert_types as et
    E, X, K, F, T, types, path = draw_slot(seed)
    print(f"[case] random slot seed {seed}: E={E} X={X} K={K} F={F} T={T} types={types} path={path}", flush=True)
    L = et.typed_layer(E, X, K, F, types, seed)
    x = orc.make_input(E, T, seed, rmsnorm=True)
    exact = path == "fp32"
    ref_out, ref = L.moe(x, debug=True, exact=exact)
    with q.Context(E, X, K, F, n_layer=1, max_tokens=T) as ctx:
        ctx.upload(0, L.router, (types[0], L.gate), (types[1], L.up), (types[2], L.down))
        ctx.set_path({"auto": q.PATH_AUTO, "exact": q.PATH_EXACT, "mfma": q.PATH_MFMA, "fp32": q.PATH_FP32}[path])
        out, got = ctx.moe_debug(0, x)
        out2 = ctx.moe(0, x)
    for k in ("sel", "start", "slot_t", "slot_of", "active"):
        assert np.array_equal(got[k], ref[k]), k
    keys = ("logits", "wt", "gu", "act", "dn") if exact else ("logits", "wt", "xq", "gu", "act", "aq", "dn")
    for k in keys:
        assert np.array_equal(_bits(got[k]), _bits(ref[k])), k
    assert np.array_equal(_bits(out), _bits(ref_out)), "layer output"
    assert np.array_equal(_bits(out2), _bits(ref_out)), "second call"
