"""Layers built so that the expert kernels' own fp32 outputs are per-block int32 dots, exactly.

Each expert row has one designated 32-block b*(expert, row) with a non-zero scale; every other
block of the row has scale 0 (and for Q4_1 offset m 0; for Q6_K the other super-blocks' d and
the other sub-scales 0), so the row's chain (src/kernels.c:85-94, 113-120, 142-170) adds the
designated block's lane sums and nothing else. Scales are powers of two chosen so that every
product and sum of the chain is exact in fp32:

* gate/up probe: the layer input holds k/128 with |k| <= 127 and one 127 per block, so each
  block quantises with d = 2^-7 and codes k; with the row scale 1, gate and up rows equal
  2^-7 * (the block's int32 dot).
* down probe: input blocks 0 and 1 hold the fixed pattern (127, 1, ..., 1)/128 in every token.
  Gate rows read block 0 with scale 16 and codes whose dot is 1024, so every gate value is 128,
  silu(128) = 128 exactly (expf(-128) is 0) and act = 128 * up. Up rows read block 1 with
  scale 1 and codes whose dot is 1016 on one row of each 32-row group and below 1016 in
  magnitude on the others, so act equals the up dot and every activation block quantises with
  d = 1016/127 = 8. Down rows, scale 1/8, then equal the down block's int32 dot against the
  activation block.

The oracle's own chain is checked to give these values (tests/test_probe_layers.py) before the device
is compared with them, and with the reference's moe() where its build is present."""
from __future__ import annotations

import copy

import numpy as np

import oracle as orc

F16_ONE, F16_16, F16_EIGHTH = 0x3C00, 0x4C00, 0x3000
PATTERN = np.array([127] + [1] * 31, np.int64)          # codes of the fixed down-probe input blocks


def designated(X: int, rows: int, nb: int, salt: int) -> np.ndarray:
    """b*(expert, row): [X][rows] block indices spread over every block position."""
    e = np.arange(X, dtype=np.int64)[:, None]
    r = np.arange(rows, dtype=np.int64)[None, :]
    return ((7 * r + 3 * e + salt) % nb).astype(np.int32)


def _random_bytes(rng, n: int) -> np.ndarray:
    return rng.integers(0, 2 ** 63, size=n // 8 + 1, dtype=np.uint64).view(np.uint8)[:n]


def _set_codes_q4(blocks: np.ndarray, off: int, codes: np.ndarray):
    """Write 32 4-bit codes per block (element j < 16: low nibble of byte j, else high nibble of
    byte j - 16) into blocks[..., off:off+16]."""
    lo, hi = codes[..., :16].astype(np.uint8), codes[..., 16:].astype(np.uint8)
    blocks[..., off:off + 16] = lo | (hi << 4)


def crafted_rows(t: int, X: int, rows: int, cols: int, bstar: np.ndarray, scale_f16: int, rng,
                 codes: np.ndarray | None = None) -> np.ndarray:
    """Stacked expert tensor [X][rows] of type t: random codes, scale scale_f16 on block
    bstar[e][r] of each row and 0 elsewhere. codes ([X][rows][32], optional): the designated
    block's codes (Q4_0 / Q4_1 only)."""
    nb = cols // 32
    if t in (orc.T_Q4_0, orc.T_Q4_1):
        bb = 18 if t == orc.T_Q4_0 else 20
        w = _random_bytes(rng, X * rows * nb * bb).reshape(X, rows, nb, bb)
        w[..., 0:bb - 16] = 0                                   # d (and m) of every block
        e, r = np.meshgrid(np.arange(X), np.arange(rows), indexing="ij")
        sel = w[e, r, bstar]                                    # [X][rows][bb] copy of b*
        sel[..., 0] = scale_f16 & 0xFF
        sel[..., 1] = scale_f16 >> 8
        if codes is not None:
            _set_codes_q4(sel, bb - 16, codes)
        w[e, r, bstar] = sel
        return w.reshape(-1)
    assert t == orc.T_Q6_K and codes is None
    nsb = cols // 256
    w = _random_bytes(rng, X * rows * nsb * 210).reshape(X, rows, nsb, 210)
    w[..., 192:210] = 0                                         # sub-scales and d
    e, r = np.meshgrid(np.arange(X), np.arange(rows), indexing="ij")
    sb = bstar // 8
    sel = w[e, r, sb]
    sel[..., 208] = scale_f16 & 0xFF
    sel[..., 209] = scale_f16 >> 8
    half, g = (bstar % 8) // 4, bstar % 4
    sc = rng.integers(-15, 16, size=(X, rows, 2)).astype(np.int8).view(np.uint8)
    idx = 192 + 8 * half + 2 * g
    np.put_along_axis(sel, idx[..., None], sc[..., :1], axis=-1)
    np.put_along_axis(sel, (idx + 1)[..., None], sc[..., 1:], axis=-1)
    w[e, r, sb] = sel
    return w.reshape(-1)


def probe_input(E: int, T: int, seed: int, fixed_blocks: int = 0) -> np.ndarray:
    """[T][E] values k/128, |k| <= 127, element 0 of every block 127 (so every block quantises
    with d = 2^-7 and codes k); the first fixed_blocks blocks hold PATTERN/128 in every token."""
    rng = np.random.default_rng(seed)
    k = rng.integers(-127, 128, size=(T, E // 32, 32))
    k[..., 0] = 127
    k[:, :fixed_blocks, :] = PATTERN
    return (k.astype(np.float32) / np.float32(128.0)).reshape(T, E)


def _codes_with_dot(rng, n: int, c0: int, rest: int) -> np.ndarray:
    """[n][32] codes with c[0] = c0 and sum_{j>=1} (c_j - 8) = rest, at random positions."""
    assert 0 <= rest <= 31 * 7
    full, part = divmod(rest, 7)
    codes = np.full((n, 32), 8, np.int64)
    codes[:, 0] = c0
    order = np.argsort(rng.random((n, 31)), axis=1) + 1        # a random order of positions 1..31
    rows = np.arange(n)[:, None]
    codes[rows, order[:, :full]] = 15
    if part:
        codes[np.arange(n), order[:, full]] = 8 + part
    return codes


def _router(E: int, X: int, seed: int, col0) -> np.ndarray:
    r = (np.random.default_rng(seed).standard_normal((X, E)) * 0.035).astype(np.float32)
    if col0 is not None:
        r[:, 0] = col0
    return r


def _host_layer(E, X, K, F, types, router, gate, up, down) -> orc.Layer:
    L = orc.Layer(E, X, K, F, 1, gate_type=types[0], up_type=types[1], down_type=types[2], experts=[])
    L.router = np.ascontiguousarray(router, np.float32)
    L.gate, L.up, L.down = gate, up, down
    L.have = set(range(X))
    return L


def gateup_probe(E, X, K, F, seed, gate_type=orc.T_Q4_0, up_type=orc.T_Q4_0, router_col0=None):
    """(layer, bstar_gate, bstar_up): gate and up rows are 2^-7 x their designated block dot on
    probe_input."""
    rng = np.random.default_rng(seed)
    bg, bu = designated(X, F, E // 32, 1), designated(X, F, E // 32, 5)
    gate = crafted_rows(gate_type, X, F, E, bg, F16_ONE, rng)
    up = crafted_rows(up_type, X, F, E, bu, F16_ONE, rng)
    down = crafted_rows(orc.T_Q4_0, X, E, F, designated(X, E, F // 32, 3), F16_EIGHTH, rng)
    return _host_layer(E, X, K, F, (gate_type, up_type, orc.T_Q4_0), _router(E, X, seed, router_col0),
                       gate, up, down), bg, bu


def down_probe(E, X, K, F, seed, down_type=orc.T_Q4_0, router_col0=None):
    """(layer, bstar_down): on probe_input(..., fixed_blocks=2) every gate value is 128, act is
    the up dot, every activation block has d = 8, and down rows are their designated block dot."""
    rng = np.random.default_rng(seed)
    gcodes = _codes_with_dot(rng, X * F, 15, 135).reshape(X, F, 32)          # dot 127*7 + 135 = 1024
    ucodes = rng.integers(0, 16, size=(X, F, 32))
    ucodes[..., 0] = rng.integers(5, 12, size=(X, F))                          # |dot| <= 3*127 + 248 < 1016
    top = rng.integers(0, 32, size=(X, F // 32))                               # one row per 32 at 1016
    g_rows = (np.arange(F // 32) * 32)[None, :] + top
    ucodes[np.arange(X)[:, None], g_rows] = _codes_with_dot(rng, X * (F // 32), 15, 127).reshape(X, F // 32, 32)
    gate = crafted_rows(orc.T_Q4_0, X, F, E, np.zeros((X, F), np.int32), F16_16, rng, gcodes)
    up = crafted_rows(orc.T_Q4_0, X, F, E, np.ones((X, F), np.int32), F16_ONE, rng, ucodes)
    bd = designated(X, E, F // 32, 2)
    down = crafted_rows(down_type, X, E, F, bd, F16_EIGHTH, rng)
    return _host_layer(E, X, K, F, (orc.T_Q4_0, orc.T_Q4_0, down_type), _router(E, X, seed, router_col0),
                       gate, up, down), bd


def with_router_col0(L: orc.Layer, col0) -> orc.Layer:
    """The same layer (expert bytes shared) with router column 0 replaced, or L itself."""
    if col0 is None:
        return L
    M = copy.copy(L)
    M.router = L.router.copy()
    M.router[:, 0] = col0
    return M


def slot_experts(start: np.ndarray, NS: int) -> np.ndarray:
    return (np.searchsorted(start, np.arange(NS), side="right") - 1).astype(np.int32)


def expected_gateup(L: orc.Layer, bg, bu, dbg) -> np.ndarray:
    """[NS][2F] 2^-7 x the designated block dots of each slot's gate and up rows."""
    E, F = L.E, L.F
    NS = dbg["slot_t"].shape[0]
    ex = np.repeat(slot_experts(dbg["start"], NS), F)
    row = np.tile(np.arange(F, dtype=np.int32), NS)
    xrow = np.repeat(dbg["slot_t"].astype(np.int64) * (E // 32), F)
    out = np.empty((NS, 2 * F), np.float32)
    for h, (w, b, t) in enumerate(((L.gate, bg, L.types[0]), (L.up, bu, L.types[1]))):
        dots = orc.block_dots_at(t, w, L.rb[h], L.eb[h], ex, row, b[ex, row], dbg["xq"], xrow)
        out[:, h * F:(h + 1) * F] = (dots.astype(np.float32) / np.float32(128.0)).reshape(NS, F)
    return out


def expected_down(L: orc.Layer, bd, dbg) -> np.ndarray:
    """[NS][E] the designated down block dots of each slot against its activation blocks."""
    E, F = L.E, L.F
    NS = dbg["slot_t"].shape[0]
    ex = np.repeat(slot_experts(dbg["start"], NS), E)
    row = np.tile(np.arange(E, dtype=np.int32), NS)
    xrow = np.repeat(np.arange(NS, dtype=np.int64) * (F // 32), E)
    dots = orc.block_dots_at(L.types[2], L.down, L.rb[2], L.eb[2], ex, row, bd[ex, row], dbg["aq"], xrow)
    return dots.astype(np.float32).reshape(NS, E)
