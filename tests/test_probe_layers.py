"""The block-dot probe layers (tests/probe_layers.py) on the CPU: in the oracle's chain (and in
the reference's moe() where its build is present) gate/up rows come out as 2^-7 x the
designated block's int32 dot and down rows as the down block's int32 dot, bit for bit. The GPU
test (test_gpu_block_dots.py) then holds the device kernels to the same values."""
import numpy as np
import pytest

import oracle as orc
import probe_layers as pl

SMALL = dict(E=256, X=16, K=4, F=256)


def _bits(a):
    return np.ascontiguousarray(a).view(np.uint32)


@pytest.mark.parametrize("types", [(orc.T_Q4_0, orc.T_Q4_0), (orc.T_Q4_1, orc.T_Q6_K), (orc.T_Q6_K, orc.T_Q4_1)])
def test_gateup_probe_rows_are_block_dots(types):
    L, bg, bu = pl.gateup_probe(**SMALL, seed=3, gate_type=types[0], up_type=types[1])
    x = pl.probe_input(SMALL["E"], 8, 11)
    out, d = L.moe(x, debug=True)
    assert np.all(d["xq"]["d"] == np.float32(2.0 ** -7))
    exp = pl.expected_gateup(L, bg, bu, d)
    assert np.array_equal(_bits(d["gu"]), _bits(exp))
    assert np.count_nonzero(exp) > 0.9 * exp.size                  # the dots are not trivially 0
    R = orc.load_ref()
    if R is not None:
        assert np.array_equal(_bits(orc.ref_moe(R, L, x)), _bits(out))


@pytest.mark.parametrize("dt", [orc.T_Q4_0, orc.T_Q4_1, orc.T_Q6_K])
def test_down_probe_rows_are_block_dots(dt):
    E, F = SMALL["E"], SMALL["F"]
    L, bd = pl.down_probe(**SMALL, seed=4, down_type=dt)
    x = pl.probe_input(E, 8, 12, fixed_blocks=2)
    out, d = L.moe(x, debug=True)
    assert np.all(d["gu"][:, :F] == 128.0)
    assert np.all(d["aq"]["d"] == 8.0)
    assert np.all(np.abs(d["act"]).reshape(-1, F // 32, 32).max(axis=2) == 1016.0)
    exp = pl.expected_down(L, bd, d)
    assert np.array_equal(_bits(d["dn"]), _bits(exp))
    assert np.count_nonzero(exp) > 0.9 * exp.size
    R = orc.load_ref()
    if R is not None:
        assert np.array_equal(_bits(orc.ref_moe(R, L, x)), _bits(out))


def test_probe_detects_a_wrong_block():
    """A dot taken at a neighbouring block does not match: the designated block is what counts."""
    L, bg, bu = pl.gateup_probe(**SMALL, seed=5)
    x = pl.probe_input(SMALL["E"], 4, 13)
    _, d = L.moe(x, debug=True)
    wrong = pl.expected_gateup(L, (bg + 1) % (SMALL["E"] // 32), bu, d)
    F = SMALL["F"]
    assert not np.array_equal(_bits(d["gu"][:, :F]), _bits(wrong[:, :F]))
