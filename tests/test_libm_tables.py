"""The tables of the kernels' expf and exp (large_model_amd/csrc/qmsg_libm.h) recomputed here from
their definition with exact decimal arithmetic.

The expf table holds 2^(i/32) rounded to double, minus i << 47 in its bit pattern; the exp table
holds for each i the relative tail 2^(i/128)/H - 1 rounded to double and H = 2^(i/128) rounded to
double, minus i << 45. Python's float(Decimal) rounds correctly, and 60 significant digits leave
no rounding in doubt for these values.
"""
import os
import re
import struct
from decimal import Decimal, getcontext

HDR = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "large_model_amd", "csrc",
                   "qmsg_libm.h")


def _table(name: str) -> list:
    text = open(HDR).read()
    m = re.search(name + r"\[(\d+)\]\s*=\s*\{(.*?)\};", text, re.S)
    assert m, name
    vals = [int(v, 16) for v in re.findall(r"0x([0-9a-fA-F]+)ULL", m.group(2))]
    assert len(vals) == int(m.group(1)), name
    return vals


def _bits(f: float) -> int:
    return struct.unpack("<Q", struct.pack("<d", f))[0]


def _pow2(i: int, n: int) -> Decimal:
    return Decimal(2) ** (Decimal(i) / Decimal(n))


def test_expf_table_is_two_to_the_i_over_32():
    getcontext().prec = 60
    tab = _table("kQmsgExp2fTab")
    for i in range(32):
        h = float(_pow2(i, 32))
        assert tab[i] == (_bits(h) - (i << 47)) & (2**64 - 1), i


def test_exp_table_is_two_to_the_i_over_128_with_tails():
    getcontext().prec = 60
    tab = _table("kQmsgExpTab")
    for i in range(128):
        v = _pow2(i, 128)
        h = float(v)
        tail = float(v / Decimal(h) - 1)
        assert tab[2 * i] == _bits(tail), i
        assert tab[2 * i + 1] == (_bits(h) - (i << 45)) & (2**64 - 1), i
