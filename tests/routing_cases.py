"""Routing edge cases shared by the CPU and GPU tests: a non-finite logit, and an exact logit
tie at the top-K boundary with probabilities that underflow to zero.

Each case is a tiny layer (E 256, X 16, K 4, F 128) whose router column 0 is replaced and whose
inputs put a chosen value in column 0, so the logits of the interesting experts are known
exactly. `expect_sel` is what the reference's K rounds of argmax (src/model.c:1053-1062)
give by hand: p compares with strict `>`, so NaN probabilities never win and equal ones go to
the lower index.
"""
import numpy as np

import oracle as orc

E, X, K, F = 256, 16, 4, 128


def nonfinite_case(seed=81):
    """Token 0: expert 5's logit is 1.5e38, all others are finite and far below, so p5 = 1 and
    every other p underflows to 0: sel = [5, 0, 1, 2]. Token 1: the same router weight times
    2.0 overflows to +inf, mx = inf and exp(inf - inf) is NaN, so z and every p are NaN and
    the argmax rounds take experts 0 .. K-1 with NaN weights."""
    col0 = orc.synth_f32(seed, 0, orc.KIND_ROUTER, 0, X * E, 0.02).reshape(X, E)[:, 0].copy()
    col0[5] = np.float32(3e38)
    x = orc.make_input(E, 2, seed)
    x[0, 0] = 0.5
    x[1, 0] = 2.0
    expect_sel = np.array([[5, 0, 1, 2], [0, 1, 2, 3]], np.int32)
    return col0, x, expect_sel


def boundary_underflow_case(seed=82):
    """One token equal to the unit vector e_0, so logit_e = col0[e] exactly. Experts 10, 11, 12
    lead (2000, 1999, 1998); experts 13 and 14 tie at 1000 and expert 2 sits at 500, all three
    more than 745 below the maximum, so their p (and every other p) is exactly 0. The
    reference takes the lowest untaken index for the fourth pick, expert 0, not expert 13 that
    leads the logit order at the boundary."""
    col0 = np.zeros(X, np.float32)
    col0[10], col0[11], col0[12] = 2000.0, 1999.0, 1998.0
    col0[13] = col0[14] = 1000.0
    col0[2] = 500.0
    x = np.zeros((1, E), np.float32)
    x[0, 0] = 1.0
    expect_sel = np.array([[10, 11, 12, 0]], np.int32)
    return col0, x, expect_sel


CASES = {"nonfinite": nonfinite_case, "boundary_underflow": boundary_underflow_case}


def layer(col0, seed):
    return orc.Layer(E, X, K, F, seed, experts=[], router_col0=col0)


def same_bits_or_both_nan(a, b) -> bool:
    """Float arrays equal bit for bit where finite or infinite, NaN in the same places (the
    sign and payload of a NaN differ between x86 and the GPU's default NaN)."""
    a = np.ascontiguousarray(a, np.float32)
    b = np.ascontiguousarray(b, np.float32)
    na, nb = np.isnan(a), np.isnan(b)
    return bool(np.array_equal(na, nb) and np.array_equal(a[~na].view(np.uint32), b[~nb].view(np.uint32)))
