"""The MFMA expert kernels (f16 MFMA lane sums + the reference's fp32 chains on the VALU) on the
GPU: every intermediate bit for bit against the oracle, like the exact path.

The MFMA kernels run for QMSG_PATH_MFMA at any batch of two or more tokens; the default path
takes them for gate/up from 1.25 slots per active expert and for down from 64 slots (Q6_K
down rows: 32), so the 16-token and the 8-token Q6_K cases also run the row-kernel gate/up
followed by the MFMA down.
The block shapes (4-, 8- and 16-slot blocks, and the Q4 waves of 16 slots from 8 slots per
expert, chosen per kernel by slots per expert) are all covered. Cases cover Q4_0 / Q4_1 /
Q6_K down rows, tiles of up to 32 slots run as 16-slot blocks, odd slot
counts per expert, the Zipf-skewed 512-token prefill, shapes whose down rows fall back to the
exact kernel (F/32 not a whole number of 8-block chunks), and batches of alternating sizes on
one context."""
import numpy as np
import pytest

import oracle as orc

pytestmark = pytest.mark.gpu

CASES = [
    # name, E, X, K, F, T, seed, down_type, zipf
    ("q30b_t64", 2048, 128, 8, 768, 64, 1, orc.T_Q4_0, False),
    ("q30b_t128", 2048, 128, 8, 768, 128, 11, orc.T_Q4_0, False),    # 8 slots per expert: 16-slot waves from here
    ("q235b_t64", 4096, 128, 8, 1536, 64, 2, orc.T_Q4_0, False),
    ("q235b_t16", 4096, 128, 8, 1536, 16, 12, orc.T_Q4_0, False),    # about one slot per expert
    ("q235b_t33", 4096, 128, 8, 1536, 33, 3, orc.T_Q4_0, False),
    ("q235b_q6k_t64", 4096, 128, 8, 1536, 64, 6, orc.T_Q6_K, False),
    ("q235b_q6k_t8", 4096, 128, 8, 1536, 8, 13, orc.T_Q6_K, False),   # Q6_K down on MFMA below one slot
    ("q235b_q41_t64", 4096, 128, 8, 1536, 64, 7, orc.T_Q4_1, False),
    ("q235b_q41_t24", 4096, 128, 8, 1536, 24, 14, orc.T_Q4_1, False),  # 4-slot blocks, Q4_1 down
    ("q480b_t48", 6144, 160, 8, 2560, 48, 8, orc.T_Q4_0, False),
    ("tiny_t40", 256, 16, 4, 128, 40, 9, orc.T_Q4_0, False),         # down on the exact kernel
    ("tiny_q6k_t200", 256, 16, 4, 256, 200, 10, orc.T_Q6_K, False),  # 50 slots per expert: 16-slot blocks
    ("q30b_q41_t256", 2048, 128, 8, 768, 256, 15, orc.T_Q4_1, False),  # 16 slots per expert: wide Q4_1 down
    # 16-slot blocks on one, two and three staged chunks (n_embd / 256 for gate/up, n_ff_exp / 256
    # for down): the double-buffered weights' first and last chunks
    ("tiny_t200", 256, 16, 4, 256, 200, 16, orc.T_Q4_0, False),
    ("small_t160", 512, 16, 4, 512, 160, 17, orc.T_Q4_1, False),
    ("small_t96", 768, 16, 4, 768, 96, 18, orc.T_Q4_0, False),
    ("q235b_zipf_t512", 4096, 128, 8, 1536, 512, 5, orc.T_Q4_0, True),
]


@pytest.fixture(scope="module")
def q():
    from large_model_amd import qmsg
    return qmsg


def _bits(a):
    return np.ascontiguousarray(a).view(np.uint8)


@pytest.mark.parametrize("name,E,X,K,F,T,seed,dt,zipf", CASES, ids=[c[0] for c in CASES])
def test_mfma_bit_exact(q, name, E, X, K, F, T, seed, dt, zipf):
    from large_model_amd.workloads import zipf_bias
    print(f"[case] mfma {name} T={T} down={dt}", flush=True)
    col0 = zipf_bias(X, K, T, E) if zipf else None
    x = orc.make_input(E, T, seed, bias_col0=zipf)
    host = orc.Layer(E, X, K, F, seed, down_type=dt, experts=[], router_col0=col0)
    ref_out, ref = host.moe(x, debug=True)
    with q.Context(E, X, K, F, n_layer=1, max_tokens=T) as ctx:
        ctx.synth(0, seed, down_type=dt, router_col0=col0)
        ctx.set_path(q.PATH_MFMA)
        out, got = ctx.moe_debug(0, x)
        ctx.set_path(q.PATH_AUTO)        # per stage: row kernels or MFMA by slots per expert
        out_auto, got_auto = ctx.moe_debug(0, x)
    for path, o, g in (("mfma", out, got), ("default", out_auto, got_auto)):
        for k in ("sel", "start", "slot_t", "slot_of", "active"):
            assert np.array_equal(g[k], ref[k]), (path, k)
        for k in ("logits", "wt", "xq", "gu", "act", "aq", "dn"):
            assert np.array_equal(_bits(g[k]), _bits(ref[k])), (path, k)
        assert np.array_equal(_bits(o), _bits(ref_out)), (path, "layer output")


def test_mfma_repeated_calls_and_sizes(q):
    """Alternating batch sizes on one context (tile lists rebuilt each call), MFMA against the
    exact path bit for bit."""
    E, X, K, F = 2048, 128, 8, 768
    with q.Context(E, X, K, F, n_layer=1, max_tokens=96) as ctx:
        ctx.synth(0, 9)
        for T in (96, 33, 2, 64, 70):
            x = orc.make_input(E, T, 40 + T)
            ctx.set_path(q.PATH_EXACT)
            ref = ctx.moe(0, x)
            ctx.set_path(q.PATH_MFMA)
            out = ctx.moe(0, x)
            assert np.array_equal(_bits(out), _bits(ref)), T


GATE_UP_CASES = [
    # name, E, X, K, F, T, seed, gate/up type, down type
    ("q235b_gq41_t24", 4096, 128, 8, 1536, 24, 31, orc.T_Q4_1, orc.T_Q4_0),     # 4-slot blocks
    ("q235b_gq41_t64", 4096, 128, 8, 1536, 64, 32, orc.T_Q4_1, orc.T_Q6_K),     # 8-slot blocks
    ("q30b_gq41_t256", 2048, 128, 8, 768, 256, 33, orc.T_Q4_1, orc.T_Q4_1),     # 16-slot blocks
    ("q235b_gq6k_t24", 4096, 128, 8, 1536, 24, 34, orc.T_Q6_K, orc.T_Q4_0),     # Q6_K gate/up, 4-slot
    ("q235b_gq6k_t64", 4096, 128, 8, 1536, 64, 35, orc.T_Q6_K, orc.T_Q6_K),     # 8-slot blocks
    ("q30b_gq6k_t256", 2048, 128, 8, 768, 256, 36, orc.T_Q6_K, orc.T_Q4_1),     # 16-slot blocks
]


@pytest.mark.parametrize("name,E,X,K,F,T,seed,gt,dt", GATE_UP_CASES, ids=[c[0] for c in GATE_UP_CASES])
def test_mfma_gateup_types_bit_exact(q, name, E, X, K, F, T, seed, gt, dt):
    """Q4_1 gate and up rows on the MFMA kernels (unsigned codes, the offset chain
    off = fma(m, ds, off), src/kernels.c:113-120) and Q6_K ones (6-bit codes, sub-scales, the
    32-scaled offset chain, src/kernels.c:142-170): every intermediate against the oracle."""
    print(f"[case] mfma gate/up {name} T={T}", flush=True)
    x = orc.make_input(E, T, seed)
    host = orc.Layer(E, X, K, F, seed, gate_type=gt, up_type=gt, down_type=dt, experts=[])
    ref_out, ref = host.moe(x, debug=True)
    with q.Context(E, X, K, F, n_layer=1, max_tokens=T) as ctx:
        ctx.synth(0, seed, gate_type=gt, up_type=gt, down_type=dt)
        results = []
        for path in (q.PATH_MFMA, q.PATH_AUTO):
            ctx.set_path(path)
            results.append(ctx.moe_debug(0, x))
    for o, g in results:
        for k in ("sel", "start", "slot_t", "slot_of", "active"):
            assert np.array_equal(g[k], ref[k]), k
        for k in ("logits", "wt", "xq", "gu", "act", "aq", "dn"):
            assert np.array_equal(_bits(g[k]), _bits(ref[k])), k
        assert np.array_equal(_bits(o), _bits(ref_out)), "layer output"


SCALE_CASES = [
    # name, scale of every other token, gate type, up type, down type
    ("acts_subnormal_q4_0", 1e-20, orc.T_Q4_0, orc.T_Q4_0, orc.T_Q4_0),   # activation blocks' d ~1e-43
    ("input_tiny_q4_0", 1e-36, orc.T_Q4_0, orc.T_Q4_0, orc.T_Q4_0),       # input blocks' d ~1e-38
    ("acts_subnormal_q4_1", 1e-20, orc.T_Q4_1, orc.T_Q4_1, orc.T_Q4_1),
    ("input_tiny_q4_1", 1e-36, orc.T_Q4_1, orc.T_Q4_1, orc.T_Q6_K),
    ("input_tiny_q6_k", 1e-36, orc.T_Q6_K, orc.T_Q6_K, orc.T_Q6_K),
    # gate and up of different types take the row kernels, so the MFMA down kernel's records
    # come from act_quant_kernel, which must flag the out-of-range ones itself
    ("acts_subnormal_rowgu_q4_0", 1e-20, orc.T_Q4_1, orc.T_Q4_0, orc.T_Q4_0),
    ("acts_subnormal_rowgu_q4_1", 1e-20, orc.T_Q4_0, orc.T_Q4_1, orc.T_Q4_1),
]


@pytest.mark.parametrize("name,scale,gt,ut,dt", SCALE_CASES, ids=[c[0] for c in SCALE_CASES])
def test_mfma_scale_ranges(q, name, scale, gt, ut, dt):
    """Blocks whose d_x lies outside [2^-102, 2^88], where fl(d_w d_x 2^24) can differ from
    fl(d_w d_x) 2^24 (subnormal products): the Q4 MFMA kernels must take their unscaled loop
    for such launches, Q6_K needs no range. Every other token is scaled down, so a launch mixes
    in-range and out-of-range records. Checked: the case does put records out of range."""
    E, X, K, F, T, seed = 2048, 128, 8, 768, 64, 41
    print(f"[case] mfma scale range {name}", flush=True)
    x = orc.make_input(E, T, seed)
    x[1::2] *= np.float32(scale)
    host = orc.Layer(E, X, K, F, seed, gate_type=gt, up_type=ut, down_type=dt, experts=[])
    ref_out, ref = host.moe(x, debug=True)
    d = np.concatenate([ref["xq"]["d"].ravel(), ref["aq"]["d"].ravel()])
    assert ((d != 0) & ((d < 2.0 ** -102) | (d > 2.0 ** 88))).any(), "no record outside the range"
    if gt != ut:
        da = ref["aq"]["d"].ravel()
        assert ((da != 0) & (da < 2.0 ** -102)).any(), "no activation record outside the range"
    with q.Context(E, X, K, F, n_layer=1, max_tokens=T) as ctx:
        ctx.synth(0, seed, gate_type=gt, up_type=ut, down_type=dt)
        results = []
        for path in (q.PATH_MFMA, q.PATH_AUTO):
            ctx.set_path(path)
            results.append(ctx.moe_debug(0, x))
        # the same context on in-range inputs next: no flag of this call may linger
        x2 = orc.make_input(E, T, seed + 1)
        ref2 = host.moe(x2)
        ctx.set_path(q.PATH_MFMA)
        out2 = ctx.moe(0, x2)
    for o, g in results:
        for k in ("sel", "start", "slot_t", "slot_of", "active"):
            assert np.array_equal(g[k], ref[k]), k
        for k in ("logits", "wt", "xq", "gu", "act", "aq", "dn"):
            assert np.array_equal(_bits(g[k]), _bits(ref[k])), k
        assert np.array_equal(_bits(o), _bits(ref_out)), "layer output"
    assert np.array_equal(_bits(out2), _bits(ref2)), "in-range call after"


def _sweep_cases(n=12, seed=2026):
    """Seeded random layers for the MFMA kernels: widths, batch sizes and tensor types drawn
    from a fixed generator, so the list is the same on every run."""
    rng = np.random.default_rng(seed)
    types = [orc.T_Q4_0, orc.T_Q4_1, orc.T_Q6_K]
    out = []
    for i in range(n):
        E, F = [(2048, 768), (4096, 1536), (1024, 512)][int(rng.integers(0, 3))]
        T = int(rng.integers(5, 150))
        gt = types[int(rng.integers(0, 3))]
        dt = types[int(rng.integers(0, 3))]
        out.append((f"sweep{i}_E{E}_T{T}_g{gt}_d{dt}", E, 128, 8, F, T, 100 + i, gt, dt))
    return out


SWEEP = _sweep_cases()


@pytest.mark.parametrize("name,E,X,K,F,T,seed,gt,dt", SWEEP, ids=[c[0] for c in SWEEP])
def test_mfma_sweep(q, name, E, X, K, F, T, seed, gt, dt):
    """Seeded random shapes, batch sizes and tensor types on the forced MFMA path and the
    default path: every intermediate bit for bit against the oracle."""
    print(f"[case] mfma sweep {name}", flush=True)
    x = orc.make_input(E, T, seed)
    host = orc.Layer(E, X, K, F, seed, gate_type=gt, up_type=gt, down_type=dt, experts=[])
    ref_out, ref = host.moe(x, debug=True)
    with q.Context(E, X, K, F, n_layer=1, max_tokens=T) as ctx:
        ctx.synth(0, seed, gate_type=gt, up_type=gt, down_type=dt)
        results = []
        for path in (q.PATH_MFMA, q.PATH_AUTO):
            ctx.set_path(path)
            results.append(ctx.moe_debug(0, x))
    for o, g in results:
        for k in ("sel", "start", "slot_t", "slot_of", "active"):
            assert np.array_equal(g[k], ref[k]), k
        for k in ("logits", "wt", "xq", "gu", "act", "aq", "dn"):
            assert np.array_equal(_bits(g[k]), _bits(ref[k])), k
        assert np.array_equal(_bits(o), _bits(ref_out)), "layer output"
