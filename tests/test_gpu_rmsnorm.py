"""rmsnorm (src/model.c:403-409) on the GPU through qmsg_rmsnorm_device, bit for bit against the
oracle's sequential double chain, on rows chosen to stress the chunked ordered sum: wide
dynamic range, small integers and powers of two (many exact sums and rounding ties), leading
zeros, few mantissa bits, spikes, random exponents; rows whose length is a multiple of 512 take
the chunked sum, others (256, 132) the term-by-term one. Each row first tries the parallel
bracket of the sum and forms it in order only where the bracket leaves an output float open:
the tests run both that default and the mode that forms every row's sum in order, and rows
built to sit on a float rounding boundary check that the bracket sends them to the ordered sum."""
import numpy as np
import pytest

import oracle as orc

pytestmark = pytest.mark.gpu


def rows_of_kind(kind: int, n: int, count: int, rng) -> np.ndarray:
    shape = (count, n)
    if kind == 0:
        return rng.standard_normal(shape).astype(np.float32)
    if kind == 1:
        return (rng.standard_normal(shape) * np.exp(3.0 * rng.standard_normal(shape))).astype(np.float32)
    if kind == 2:
        return rng.integers(-3, 4, size=shape).astype(np.float32)
    if kind == 3:
        return (np.ldexp(1.0, rng.integers(-20, 20, size=shape)) * rng.choice([-1.0, 1.0], size=shape)).astype(np.float32)
    if kind == 4:
        x = rng.standard_normal(shape).astype(np.float32)
        x[:, : n // 2] = 0.0
        return x
    if kind == 5:
        return np.ldexp(1.0 + rng.integers(0, 8, size=shape) / 8.0, rng.integers(0, 6, size=shape)).astype(np.float32)
    if kind == 6:
        x = (1e-3 * rng.standard_normal(shape)).astype(np.float32)
        x[:, ::97] = (1e3 * rng.standard_normal((count, len(range(0, n, 97))))).astype(np.float32)
        return x
    bits = rng.integers(0, 2 ** 32, size=shape, dtype=np.uint64).astype(np.uint32)
    bits = (bits & np.uint32(0x807FFFFF)) | (rng.integers(100, 160, size=shape).astype(np.uint32) << np.uint32(23))
    return bits.view(np.float32)


@pytest.fixture(scope="module")
def ctx():
    from large_model_amd import qmsg
    with qmsg.Context(256, 16, 4, 128, n_layer=1, max_tokens=1) as c:
        yield c


# 512-multiples take the chunked sum: up to 8192 floats the row stays held in registers, above
# that (12288, 16384) the kernel loops over several bases and rereads the row for the output,
# and 16384 has 256 chunks per row. 132, 256 and 9004 take the term-by-term sum.
@pytest.mark.parametrize("walk", [False, True], ids=["bracket", "walk"])
@pytest.mark.parametrize("n", [256, 2048, 4096, 6144, 7168, 12288, 16384, 132, 9004])
def test_rmsnorm_rows_bit_exact(ctx, n, walk):
    print(f"[case] rmsnorm n={n} walk={walk}", flush=True)
    rng = np.random.default_rng(n)
    x = np.concatenate([rows_of_kind(k, n, 24, rng) for k in range(8)])
    w = rng.uniform(0.5, 1.5, n).astype(np.float32)
    ctx.rmsnorm_mode(walk)
    try:
        for weights in (None, w):
            ref = orc.rmsnorm(x, weights, eps=1e-6)
            for inplace in (True, False):
                got = ctx.rmsnorm(x, weights, eps=1e-6, inplace=inplace)
                assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)), (n, weights is None, inplace)
        walked = ctx.rmsnorm_mode(False)
        if walk:
            assert walked == 4 * x.shape[0]
        else:
            assert walked < x.shape[0]
    finally:
        ctx.rmsnorm_mode(False)


def rows_on_a_boundary(n: int, count: int, rng, eps: float = 1e-6) -> np.ndarray:
    """Rows whose output hangs on the last bits of ss: standard normal elements, and a last one
    of magnitude below 2^-24, whose square (below 2^-48) leaves the sequential sum as it was,
    with the 24-bit mantissa that puts x * inv closest to the midpoint of two floats; a row is
    kept when that is within 2e-14 of it, relative (the bracket's half-width is about 1e-13)."""
    rows = []
    m = np.arange(2 ** 23, 2 ** 24, dtype=np.float64)
    v = m * 2.0 ** -48                                          # floats in [2^-25, 2^-24)
    while len(rows) < count:
        x = rng.standard_normal(n).astype(np.float32)
        x[-1] = 0.0
        sq = x.astype(np.float64) * x.astype(np.float64)
        ss = np.add.accumulate(sq)[-1]                          # in index order
        assert ss > 2.0 ** -6, "the last square must stay below half an ulp of ss"
        inv = 1.0 / np.sqrt(ss / n + np.float64(np.float32(eps)))
        p = v * inv
        ulp = np.ldexp(1.0, np.frexp(p)[1] - 24)                # float spacing at p
        units = p / ulp
        dist = np.abs(units - np.floor(units) - 0.5) * ulp / p
        best = int(np.argmin(dist))
        if dist[best] < 2e-14:
            x[-1] = np.float32(v[best])
            rows.append(x)
    return np.stack(rows)


@pytest.mark.parametrize("n", [4096, 16384, 9004])
def test_rmsnorm_rows_on_a_boundary(ctx, n):
    print(f"[case] rmsnorm on a rounding boundary n={n}", flush=True)
    rng = np.random.default_rng(100 + n)
    x = rows_on_a_boundary(n, 6, rng)
    ctx.rmsnorm_mode(False)
    got, ref = ctx.rmsnorm(x), orc.rmsnorm(x, eps=1e-6)
    assert ctx.rmsnorm_mode(False) == x.shape[0], "every such row must form its sum in order"
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))


def test_rmsnorm_non_finite_rows(ctx):
    """An infinite or NaN element makes the sum non-finite: the kernel then adds term by term
    and matches the oracle's values (NaN where it has NaN)."""
    print("[case] rmsnorm non-finite", flush=True)
    rng = np.random.default_rng(5)
    x = rng.standard_normal((4, 4096)).astype(np.float32)
    x[0, 1000] = np.inf
    x[1, 3000] = np.nan
    x[2, 5] = -np.inf
    got, ref = ctx.rmsnorm(x), orc.rmsnorm(x)
    assert np.array_equal(np.isnan(got), np.isnan(ref))
    fin = ~np.isnan(ref)
    assert np.array_equal(got[fin].view(np.uint32), ref[fin].view(np.uint32))


def test_rmsnorm_arguments(ctx):
    from large_model_amd import qmsg
    with pytest.raises(qmsg.QmsgError):
        lib_mode = qmsg.lib.qmsg_rmsnorm_mode(ctx._h, 2, None)
        ctx._check(lib_mode)
    d = ctx.device_alloc(4096)
    with pytest.raises(qmsg.QmsgError):
        ctx.rmsnorm_device(d, d, None, 1, 6, 1e-6)            # n % 4
    with pytest.raises(qmsg.QmsgError):
        ctx.rmsnorm_device(d, d + 4, None, 1, 8, 1e-6)        # unaligned input
    with pytest.raises(qmsg.QmsgError) as ei:
        ctx.rmsnorm_device(d, d, None, 1, 1 << 16, 1e-6)      # too long for the kernel's LDS
    assert ei.value.status == -2
    ctx.rmsnorm_device(d, d, None, 0, 256, 1e-6)              # no rows: nothing to do
