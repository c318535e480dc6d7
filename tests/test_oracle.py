"""The CPU oracle against the reference's own outputs and against what the mathematics fixes.

Golden vectors in tests/golden/ come from the reference's C code (src/kernels.c, quant.c,
model.c) built by oracle/Makefile and run by tests/golden/make_golden.py. Each oracle
function is checked bit for bit against them; the planted-mistake tests show that the checks
would catch the plausible slips (operation order, nibble order, rounding, tie rule).
"""
import glob
import hashlib
import os

import numpy as np
import pytest

import oracle as orc
import routing_cases as rc

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def sha(*arrays) -> bytes:
    h = hashlib.sha256()
    for a in arrays:
        h.update(np.ascontiguousarray(a).view(np.uint8).tobytes())
    return h.digest()


def f32_bits(v):
    return np.float32(v).view(np.uint32)


@pytest.fixture(scope="module")
def kat():
    return dict(np.load(os.path.join(GOLD, "kat_kernels.npz")))


# ------------------------------------------------------------------ formats and kernels

def test_f16_known_answers():
    """tests/test_smoke.c:36-39."""
    assert orc.lib.orc_f16_to_f32(0x3C00) == 1.0
    assert orc.lib.orc_f16_to_f32(0xC000) == -2.0
    assert orc.lib.orc_f16_to_f32(0x7BFF) == 65504.0
    assert orc.lib.orc_f16_to_f32(0x0001) == 5.9604644775390625e-08


def test_f16_all_halves_match_numpy():
    """Every finite half decodes exactly (numpy's float16 is IEEE binary16)."""
    h = np.arange(0, 1 << 16, dtype=np.uint32)
    ref = h.astype(np.uint16).view(np.float16).astype(np.float32)
    got = np.array([orc.lib.orc_f16_to_f32(int(v)) for v in h[::7]], np.float32)
    fin = np.isfinite(ref[::7])
    assert np.array_equal(got[fin].view(np.uint32), ref[::7][fin].view(np.uint32))


def kernel_cases(kat):
    for i in range(int(kat["n_kernel_cases"])):
        yield (int(kat[f"k{i}_type"]), kat[f"k{i}_w"], kat[f"k{i}_x"], kat[f"k{i}_xq"], kat[f"k{i}_dot"],
               bytes(kat[f"k{i}_deq_sha"]))


def test_quantize_q8_matches_reference(kat):
    for t, w, x, xq, dot, _ in kernel_cases(kat):
        assert np.array_equal(orc.quantize_q8(x).view(np.uint8), xq)


def test_quantize_q8_ties_round_to_even(kat):
    got = orc.quantize_q8(kat["ties_x"])
    assert np.array_equal(got.view(np.uint8), kat["ties_xq"])
    q = got["q"][0].astype(int)
    # block 0 holds k - 15.5 with max 127 -> d = 1: halves round to even
    assert got["d"][0] == 1.0
    assert q[1] == -14 and q[2] == -14 and q[3] == -12


def test_quantize_q8_closed_form():
    """d = max|x|/127, q = rint(x/d), s16 = half sums, ds = d*sum; zero blocks stay zero."""
    rng = np.random.default_rng(3)
    x = rng.standard_normal(64 * 32).astype(np.float32)
    x[:32] = 0.0
    got = orc.quantize_q8(x)
    assert got["d"][0] == 0 and not got["q"][0].any() and got["ds"][0] == 0
    for b in range(1, 64):
        xb = x[32 * b:32 * b + 32]
        d = np.float32(np.abs(xb).max()) / np.float32(127.0)
        q = np.rint(xb * (np.float32(1.0) / d)).astype(np.int32)
        assert f32_bits(got["d"][b]) == f32_bits(d)
        assert np.array_equal(got["q"][b].astype(np.int32), q)
        assert got["s16"][b][0] == q[:16].sum() and got["s16"][b][1] == q[16:].sum()
        assert f32_bits(got["ds"][b]) == f32_bits(d * np.float32(q.sum()))
        assert np.abs(q).max() == 127


def test_quantize_q8_codes_outside_int():
    """Blocks whose scaled values leave int's range: d below 2^-128 (1/d = +inf), NaN and
    infinite inputs. The reference's (int)nearbyintf is x86's conversion, INT_MIN for those,
    so each such code is 0 as int8 and adds INT_MIN to its half sum (mod 2^32). Closed form
    here; bit for bit against the reference build where it is present."""
    rng = np.random.default_rng(5)
    x = rng.standard_normal((6, 32)).astype(np.float32)
    x[0] *= np.float32(1e-39)            # d below 2^-128: id = +inf
    x[1] *= np.float32(1e-44)            # subnormal inputs, the same
    x[2, 3] = np.inf                     # d = +inf, id = 0: inf * 0 is NaN
    x[3, 7] = np.nan                     # amax ignores the NaN
    x[4, :] = np.nan                     # all NaN: d = 0, every code from NaN * 0
    x[5, ::3] = -np.inf
    got = orc.quantize_q8(x.ravel())
    imin = -2 ** 31
    for b in range(6):
        xb = x[b]
        with np.errstate(all="ignore"):
            amax = np.float32(0)
            for v in xb:                 # fmaxf from 0, NaN ignored
                if not np.isnan(v):
                    amax = max(amax, np.float32(abs(v)))
            d = amax / np.float32(127)
            idv = np.float32(1) / d if d > 0 else np.float32(0)
            r = np.rint(xb * idv)
        q = np.array([int(v) if abs(v) < 2.0 ** 31 else imin for v in r], np.int64)
        assert np.array_equal(got["q"][b].astype(np.int64), ((q + 128) % 256) - 128), b
        wrap = lambda v: ((int(v) + 2 ** 31) % 2 ** 32) - 2 ** 31
        s0, s1 = wrap(q[:16].sum()), wrap(q[16:].sum())
        assert got["s16"][b][0] == ((s0 + 2 ** 15) % 2 ** 16) - 2 ** 15, b
        assert got["s16"][b][1] == ((s1 + 2 ** 15) % 2 ** 16) - 2 ** 15, b
        with np.errstate(all="ignore"):
            ds = np.float32(d) * np.float32(wrap(s0 + s1))
        assert f32_bits(got["ds"][b]) == f32_bits(ds) or (np.isnan(got["ds"][b]) and np.isnan(ds)), b
    assert not got["q"][0].any() and not got["q"][1].any()
    R = orc.load_ref()
    if R is None:
        pytest.skip("reference build (oracle/_ref) not present")
    ref = np.zeros_like(got)
    xs = np.ascontiguousarray(x.ravel())
    R.qms_quantize_q8(xs.ctypes.data, xs.size, ref.ctypes.data)
    assert np.array_equal(ref.view(np.uint8), got.view(np.uint8))


def test_vec_dot_q8_matches_reference(kat):
    for t, w, x, xq, dot, _ in kernel_cases(kat):
        n = x.size
        got = orc.vec_dot_q8(t, w, xq.view(orc.Q8_DTYPE), n)
        assert f32_bits(got) == f32_bits(dot), (t, n)


def test_dequant_matches_reference(kat):
    for t, w, x, xq, dot, deq_sha in kernel_cases(kat):
        assert sha(orc.dequant_row(t, w, x.size)) == deq_sha


def test_vec_dot_q8_invariant():
    """tests/test_kernels.c:65-83: the int8 dot equals the dequant-then-dot in double within
    1e-5 of the sum of |terms|, on the reference's own LCG cases (incl. all-zero blocks)."""
    import importlib.util
    spec = importlib.util.spec_from_file_location("mg", os.path.join(GOLD, "make_golden.py"))
    mg = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mg)
    g = mg.Lcg()
    for t in (orc.T_Q4_0, orc.T_Q4_1, orc.T_Q6_K):
        worst = 0.0
        for n in (256, 768, 1536, 2048, 4096):
            for trial in range(6):
                w = mg.fill_block(g, t, n)
                x = np.array([((g.rnd() % 20001) - 10000.0) / 3000.0 for _ in range(n)], np.float32)
                if trial % 5 == 0:
                    x[:32] = 0.0
                xq = orc.quantize_q8(x)
                wd = orc.dequant_row(t, w, n).astype(np.float64)
                xd = (xq["q"].astype(np.float64) * xq["d"][:, None].astype(np.float64)).ravel()
                ref = float(np.dot(wd, xd))
                mag = float(np.abs(wd * xd).sum())
                got = orc.vec_dot_q8(t, w, xq, n)
                worst = max(worst, abs(got - ref) / (mag + 1e-30))
        assert worst < 1e-5, (t, worst)


def brute_block_dot(t, w_row, xq, blk):
    """The exact signed int32 of a 32-block, from dequantised codes (no scales)."""
    q = xq["q"][blk].astype(np.int64)
    if t == orc.T_Q4_0:
        b = w_row[blk * 18 + 2: blk * 18 + 18].astype(np.int64)
        codes = np.concatenate([b & 15, b >> 4]) - 8
        return int((codes * q).sum())
    if t == orc.T_Q4_1:
        b = w_row[blk * 20 + 4: blk * 20 + 20].astype(np.int64)
        codes = np.concatenate([b & 15, b >> 4])
        return int((codes * q).sum())
    sb = w_row[(blk // 8) * 210:(blk // 8) * 210 + 210].astype(np.int64)
    half, g = (blk % 8) // 4, blk % 4
    ql, qh = sb[64 * half: 64 * half + 64], sb[128 + 32 * half: 128 + 32 * half + 32]
    sc = sb[192:208].astype(np.uint8).view(np.int8).astype(np.int64)[8 * half:8 * half + 8]
    lo = ql[(g & 1) * 32:(g & 1) * 32 + 32]
    nib = (lo & 15) if g < 2 else (lo >> 4)
    codes = (nib | (((qh >> (2 * g)) & 3) << 4)) - 32
    return int(sc[2 * g] * (codes[:16] * q[:16]).sum() + sc[2 * g + 1] * (codes[16:] * q[16:]).sum())


@pytest.mark.parametrize("t,n", [(orc.T_Q4_0, 1536), (orc.T_Q4_1, 1536), (orc.T_Q6_K, 1536)])
def test_block_dot_brute_force(t, n):
    L = orc.Layer(256, 16, 4, n, 9, down_type=t, experts=[3])
    x = np.random.default_rng(5).standard_normal(n).astype(np.float32)
    xq = orc.quantize_q8(x)
    row = L.down[3 * L.eb[2] + 17 * L.rb[2]: 3 * L.eb[2] + 18 * L.rb[2]]
    for blk in range(n // 32):
        assert orc.block_dot(t, row, xq, blk) == brute_block_dot(t, row, xq, blk)


def test_rmsnorm_matches_reference(kat):
    for i in range(int(kat["n_rms_cases"])):
        got = orc.rmsnorm(kat[f"r{i}_x"][None, :], kat[f"r{i}_w"])[0]
        assert np.array_equal(got.view(np.uint32), kat[f"r{i}_y"].view(np.uint32)), i


def test_device_expf_restatement_on_all_inputs():
    """The kernels' expf (qmsg_libm.h, compiled here for the CPU) equals the C library's
    expf on every one of the 2^32 float inputs."""
    assert orc.lib.orc_expf_mismatches(0, 1 << 32) == 0


def test_device_exp_restatement_sampled():
    """The kernels' double exp equals the C library's exp on 2e8 seeded inputs."""
    assert orc.lib.orc_exp_mismatches(2024, 200_000_000) == 0


def test_vec_dot_f32_matches_reference(kat):
    for i in range(int(kat["n_f32_cases"])):
        got = orc.vec_dot_f32(kat[f"f{i}_w"], kat[f"f{i}_x"])
        assert f32_bits(got) == f32_bits(kat[f"f{i}_dot"]), i


def test_silu_is_glibc():
    """SiLU is a/(1+expf(-a)) with the C library's expf (src/model.c:424)."""
    import ctypes
    libm = ctypes.CDLL("libm.so.6")
    libm.expf.restype = ctypes.c_float
    libm.expf.argtypes = [ctypes.c_float]
    for a in (-100.0, -88.5, -10.0, -1.0, -1e-3, 0.0, 1e-3, 0.5, 3.0, 20.0, 100.0):
        a = np.float32(a)
        ref = a / (np.float32(1.0) + np.float32(libm.expf(-a)))
        assert f32_bits(orc.lib.orc_silu(a)) == f32_bits(ref)


# ------------------------------------------------------------------ whole layers

def load_layer(path):
    d = dict(np.load(path))
    E, X, K, F, T, seed, dt, rms = (int(v) for v in d["shape"])
    special = str(d["special"])
    col0 = d.get("router_col0")
    gt, ut = (int(v) for v in d.get("gu_types", (orc.T_Q4_0, orc.T_Q4_0)))
    L = orc.Layer(E, X, K, F, seed, gate_type=gt, up_type=ut, down_type=dt, experts=[], router_col0=col0)
    x = orc.make_input(E, T, seed, rmsnorm=bool(rms), bias_col0=special == "zipf")
    if special == "ties":
        L.router[5] = L.router[2]
        L.router[9] = L.router[2]
    elif special == "zero":
        x[1] = 0.0
    elif special == "large":
        x *= 300.0
    return d, L, x


def check_layer(d, L, x, logits=True):
    """Raise AssertionError unless the oracle reproduces the reference's vectors."""
    assert sha(L.router) == bytes(d["router_sha"]), "router generator"
    assert sha(x) == bytes(d["x_sha"]), "input generator"
    exact = str(d["special"]) == "exact"
    lg, sel, wt = L.route(x, exact)
    if logits:
        assert sha(lg) == bytes(d["logits_sha"]), "router logits"
    xq = orc.quantize_q8(x).reshape(x.shape[0], -1)
    assert sha(xq) == bytes(d["xq_sha"]), "int8 input blocks"
    assert np.array_equal(np.unique(sel), d["experts"]), "expert ids"
    out = L.moe(x, exact=exact)
    eb = L.eb
    assert sha(*[np.concatenate([L.gate[e * eb[0]:(e + 1) * eb[0]], L.up[e * eb[1]:(e + 1) * eb[1]],
                                 L.down[e * eb[2]:(e + 1) * eb[2]]]) for e in d["experts"]]) == bytes(d["experts_sha"]), \
        "expert generator"
    if "out" in d:
        assert np.array_equal(out.view(np.uint32), d["out"].view(np.uint32)), "layer output"
    else:
        assert np.array_equal(out.ravel()[d["out_idx"]].view(np.uint32), d["out_vals"].view(np.uint32)), "layer output"
    assert sha(out) == bytes(d["out_sha"]), "layer output hash"


LAYER_FILES = sorted(glob.glob(os.path.join(GOLD, "layer_*.npz")))


@pytest.mark.parametrize("path", LAYER_FILES, ids=[os.path.basename(p)[6:-4] for p in LAYER_FILES])
def test_layer_matches_reference(path):
    d, L, x = load_layer(path)
    check_layer(d, L, x)


def test_zero_row_routes_to_lowest_experts():
    d, L, x = load_layer(os.path.join(GOLD, "layer_tiny_zero_row.npz"))
    lg, sel, wt = L.route(x)
    assert not lg[1].any()
    assert list(sel[1]) == [0, 1, 2, 3]
    assert np.all(wt[1] == np.float32(0.25))


def test_tied_experts_keep_lower_index_first():
    d, L, x = load_layer(os.path.join(GOLD, "layer_tiny_ties.npz"))
    lg, sel, wt = L.route(x)
    assert np.array_equal(lg[:, 2], lg[:, 5]) and np.array_equal(lg[:, 2], lg[:, 9])
    for t in range(x.shape[0]):
        s = list(sel[t])
        picked = [e for e in s if e in (2, 5, 9)]
        assert picked == sorted(picked)


@pytest.mark.parametrize("name", sorted(rc.CASES))
def test_routing_edge_cases(name):
    """A non-finite logit (every p NaN: experts 0 .. K-1, NaN weights) and an exact logit tie
    at the top-K boundary whose p underflow to 0 (the lowest untaken index wins): the oracle's
    selection equals the hand-derived argmax rounds, and its layer output equals the
    reference build's moe() bit for bit, NaN in the same places."""
    seed = 81 if name == "nonfinite" else 82
    col0, x, expect_sel = rc.CASES[name](seed)
    L = rc.layer(col0, seed)
    lg, sel, wt = L.route(x)
    assert np.array_equal(sel, expect_sel), sel
    if name == "nonfinite":
        assert np.isposinf(lg[1, 5]) and np.isfinite(lg[0]).all()
        assert np.isnan(wt[1]).all() and np.array_equal(wt[0], np.float32([1, 0, 0, 0]))
    else:
        assert np.array_equal(lg[0], col0)
        assert wt[0, 3] == 0.0 and np.isfinite(wt).all()
    out = L.moe(x)
    assert np.isnan(out[1]).all() if name == "nonfinite" else np.isfinite(out).all()
    R = orc.load_ref()
    if R is None:
        pytest.skip("reference build (oracle/_ref) not present")
    assert rc.same_bits_or_both_nan(orc.ref_moe(R, L, x), out)


# ------------------------------------------------------------------ shapes off the integer kernels' grid

OFF_GRID = [   # E, X, K, F, T, gate, up, down types
    (96, 8, 2, 96, 3, orc.T_Q4_0, orc.T_Q4_0, orc.T_Q4_0),
    (288, 12, 3, 160, 5, orc.T_Q4_1, orc.T_Q4_0, orc.T_Q4_1),
    (256, 16, 4, 96, 4, orc.T_Q6_K, orc.T_Q6_K, orc.T_Q4_0),
    (512, 8, 2, 32, 2, orc.T_Q4_0, orc.T_Q4_1, orc.T_Q4_0),
    (800, 10, 4, 256, 1, orc.T_Q4_0, orc.T_Q4_0, orc.T_Q6_K),
]


@pytest.mark.parametrize("E,X,K,F,T,gt,ut,dt", OFF_GRID, ids=[f"e{c[0]}_f{c[3]}" for c in OFF_GRID])
def test_off_grid_shapes(E, X, K, F, T, gt, ut, dt):
    """n_embd % 256 != 0 (the reference's moe() then runs moe_group_exact, whose qms_matmul of
    each slot takes the int8 path, src/model.c:1009-1030) and n_ff_exp = 32 x odd (its fast
    path): every slot's gate/up and down rows of the oracle's layer equal the oracle's
    qms_matmul restatement (pinned by the reference's dense fixtures) on that slot's input and
    activation row, and the layer equals the reference build's moe() bit for bit, with and
    without --exact."""
    seed = 90 + E % 97
    L = orc.Layer(E, X, K, F, seed, gate_type=gt, up_type=ut, down_type=dt, experts=[])
    x = orc.make_input(E, T, seed, rmsnorm=True)
    out, d = L.moe(x, debug=True)
    rb, eb = L.rb, L.eb
    for e in range(X):
        for s in range(int(d["start"][e]), int(d["start"][e + 1])):
            xt = x[d["slot_t"][s]][None]
            g = orc.matmul_q8(gt, L.gate[e * eb[0]:(e + 1) * eb[0]], F, E, xt)
            u = orc.matmul_q8(ut, L.up[e * eb[1]:(e + 1) * eb[1]], F, E, xt)
            assert np.array_equal(d["gu"][s].view(np.uint32), np.concatenate([g[0], u[0]]).view(np.uint32))
            dn = orc.matmul_q8(dt, L.down[e * eb[2]:(e + 1) * eb[2]], E, F, d["act"][s][None])
            assert np.array_equal(d["dn"][s].view(np.uint32), dn[0].view(np.uint32))
    R = orc.load_ref()
    if R is None:
        pytest.skip("reference build (oracle/_ref) not present")
    assert np.array_equal(orc.ref_moe(R, L, x).view(np.uint32), out.view(np.uint32))
    assert np.array_equal(orc.ref_moe(R, L, x, exact=True).view(np.uint32), L.moe(x, exact=True).view(np.uint32))


# ------------------------------------------------------------------ expert tensors of other types

Q40, Q41, Q6K, Q80, F16, F32 = orc.T_Q4_0, orc.T_Q4_1, orc.T_Q6_K, orc.T_Q8_0, orc.T_F16, orc.T_F32
TYPED = [   # E, X, K, F, T, (gate, up, down)
    (256, 16, 4, 128, 3, (Q80, Q80, Q80)),
    (256, 16, 4, 128, 1, (F16, F16, F16)),
    (256, 16, 4, 128, 4, (F32, Q40, F32)),
    (512, 8, 2, 256, 5, (Q40, Q80, Q6K)),
    (96, 8, 2, 96, 2, (Q80, Q41, F16)),
    (288, 12, 3, 96, 3, (Q40, F32, Q40)),
]


def _slot_dot_ok(t, row, x, xq, y):
    """y is row . x as the reference's qms_matmul takes it for type t: int8 blocks or dot_f32
    exactly (the dense restatement, pinned by the reference's fixtures); for F16 / Q8_0 rows
    (matmul_exact's fp32 chain) within the chain's rounding bound of the float64 dot."""
    n = x.size
    if t in (Q40, Q41, Q6K, F32):
        return np.float32(y).view(np.uint32) == orc.matmul_q8(t, row, 1, n, x[None])[0, 0].view(np.uint32)
    w = orc.dequant_row(t, row, n).astype(np.float64)
    exact = float(np.dot(w, x.astype(np.float64)))
    return abs(float(y) - exact) <= n * 2.0 ** -23 * float(np.abs(w * x).sum()) + 1e-30


@pytest.mark.parametrize("E,X,K,F,T,types", TYPED, ids=["_".join(map(str, c[5])) + f"_e{c[0]}" for c in TYPED])
def test_expert_types(E, X, K, F, T, types):
    """Q8_0, F16 and F32 expert tensors (the reference's loader takes any type; outside its fast
    gate moe_group_exact's qms_matmul picks each matrix's dot by type, src/model.c:1009-1030,
    src/quant.c:128-170): the oracle's per-slot rows follow that choice, and its layer equals
    the reference build's moe() bit for bit, with and without --exact."""
    import expert_types as et
    seed = 120 + E % 89 + T
    L = et.typed_layer(E, X, K, F, types, seed)
    x = orc.make_input(E, T, seed, rmsnorm=True)
    out, d = L.moe(x, debug=True)
    gt, ut, dt = types
    rb, eb = L.rb, L.eb
    for e in d["active"]:
        for s in range(int(d["start"][e]), int(d["start"][e + 1])):
            tk = int(d["slot_t"][s])
            for r in (0, F // 2, F - 1):
                assert _slot_dot_ok(gt, L.gate[e * eb[0] + r * rb[0]:e * eb[0] + (r + 1) * rb[0]], x[tk], None,
                                    d["gu"][s, r])
                assert _slot_dot_ok(ut, L.up[e * eb[1] + r * rb[1]:e * eb[1] + (r + 1) * rb[1]], x[tk], None,
                                    d["gu"][s, F + r])
            for r in (0, E - 1):
                assert _slot_dot_ok(dt, L.down[e * eb[2] + r * rb[2]:e * eb[2] + (r + 1) * rb[2]], d["act"][s], None,
                                    d["dn"][s, r])
    R = orc.load_ref()
    if R is None:
        pytest.skip("reference build (oracle/_ref) not present")
    assert np.array_equal(orc.ref_moe(R, L, x).view(np.uint32), out.view(np.uint32))
    assert np.array_equal(orc.ref_moe(R, L, x, exact=True).view(np.uint32), L.moe(x, exact=True).view(np.uint32))


def test_f32_up_behind_the_fast_gate_is_not_modelled():
    """Quantised gate and down with F32 up at n_embd % 256 == 0 pass the reference's fast gate,
    which sends the up rows to qms_vec_dot_q8 (no F32 case: NaN, src/kernels.c:223-231); its
    quantiser turns the NaN activations into zero blocks (d = 0), so the layer's output is all
    zeros there. The oracle refuses the layer, and the library refuses it at upload."""
    import expert_types as et
    L = et.typed_layer(256, 16, 4, 128, (Q40, F32, Q40), 77)
    x = orc.make_input(256, 2, 77, rmsnorm=True)
    with pytest.raises(RuntimeError):
        L.moe(x)
    R = orc.load_ref()
    if R is not None:
        assert not np.any(orc.ref_moe(R, L, x))


# ------------------------------------------------------------------ planted mistakes

MUTATIONS = ["HSUM_LINEAR", "CORR_UNFUSED", "NIBBLE_ORDER", "ROUTER_TREE", "ROUND_AWAY", "TIE_HIGH",
             "COMBINE_ORDER"]


@pytest.mark.parametrize("m", range(1, len(MUTATIONS) + 1), ids=MUTATIONS)
def test_planted_mistake_is_caught(m, kat):
    fast = [p for p in LAYER_FILES if "tiny" in p or "q30b" in p]
    orc.set_mutation(m)
    try:
        caught = False
        for check in (test_quantize_q8_matches_reference, test_quantize_q8_ties_round_to_even,
                      test_vec_dot_q8_matches_reference, test_vec_dot_f32_matches_reference):
            try:
                check(kat)
            except AssertionError:
                caught = True
        for p in fast:
            try:
                check_layer(*load_layer(p))
            except AssertionError:
                caught = True
        assert caught, f"mutation {MUTATIONS[m - 1]} passed every golden check"
    finally:
        orc.set_mutation(0)
