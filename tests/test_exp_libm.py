"""CPU pinning of the sampler's device exp(double) (edgeforge_amd/csrc/exp_f64.h), which must return
glibc's exp to the last bit so that sampled ids match the reference's (src/sampler.cpp:44-47).

The header's table is checked against the mathematics it states (H = nearest double to 2^(i/128),
T = (2^(i/128) - H) / H rounded, entry 2i + 1 = bits(H) - (i << 45)), computed here in 80-digit
decimal.  The header's constants and its operation order are then run in Python with every fused
multiply-add done exactly (rational arithmetic, one rounding) and compared with math.exp (the host
libm) on points that stress each branch: the rounding boundaries of k = round(x 128 / ln 2), the
rescaled ranges |x| >= 512 and the subnormal results, and random arguments.  The device itself is
swept against the host libm in tests/test_gpu_sampler.py.
"""
import math
import os
import re
import struct
from decimal import Decimal, getcontext
from fractions import Fraction

import numpy as np

HDR = os.path.join(os.path.dirname(__file__), "..", "edgeforge_amd", "csrc", "exp_f64.h")
SRC = open(HDR).read()
TABLE = [int(v, 16) for v in re.findall(r"0x([0-9a-f]{16})ull", SRC[SRC.index("kExpTable"):SRC.index("};")])]


def _const(name):
    return float.fromhex(re.search(name + r" = (-?0x[0-9a-fp.+-]+)", SRC).group(1))


def _bits(d):
    return struct.unpack("<Q", struct.pack("<d", d))[0]


def _dbl(u):
    return struct.unpack("<d", struct.pack("<Q", u & 0xFFFFFFFFFFFFFFFF))[0]


def _fma(a, b, c):
    return float(Fraction(a) * Fraction(b) + Fraction(c))


def test_table_is_the_stated_mathematics():
    assert len(TABLE) == 256
    getcontext().prec = 80
    for i in range(128):
        v = Decimal(2) ** (Decimal(i) / Decimal(128))
        hi = float(v)
        tail = float((v - Decimal(hi)) / Decimal(hi))
        assert TABLE[2 * i] == _bits(tail), i
        assert TABLE[2 * i + 1] == (_bits(hi) - (i << 45)) & 0xFFFFFFFFFFFFFFFF, i


def test_reduction_constants_are_ln2():
    getcontext().prec = 80
    ln2 = Decimal(2).ln()
    assert _const("kInvLn2N") == float(1 / ln2)  # times 128 in the header: exact
    hi = -_const("kNegLn2HiN")
    assert _bits(hi) & ((1 << 17) - 1) == 0  # a short head: k * hi is exact for |k| < 2^17
    assert -_const("kNegLn2LoN") == float(ln2 / 128 - Decimal(hi))


C2, C3, C4, C5 = (_const(n) for n in ("kC2", "kC3", "kC4", "kC5"))
INV, NHI, NLO, SHIFT = _const("kInvLn2N") * 128, _const("kNegLn2HiN"), _const("kNegLn2LoN"), _const("kShift")


def _exp(x):
    """exp_libm of the header, step for step (fused steps exact, the rest IEEE double)."""
    ux = _bits(x)
    abstop = (ux >> 52) & 0x7FF
    special = False
    if ((abstop - 0x3C9) & 0xFFFFFFFF) >= 0x408 - 0x3C9:
        if ((abstop - 0x3C9) & 0xFFFFFFFF) >= 0x80000000:
            return 1.0 + x
        if abstop >= 0x409:
            return 0.0 if ux >> 63 else math.inf
        special = True
    kd = _fma(INV, x, SHIFT)
    ki = _bits(kd)
    kd -= SHIFT
    r = _fma(kd, NLO, _fma(kd, NHI, x))
    idx = 2 * (ki % 128)
    tail = _dbl(TABLE[idx])
    sbits = (TABLE[idx + 1] + (ki << 45)) & 0xFFFFFFFFFFFFFFFF
    r2 = r * r
    tmp = _fma(r2 * r2, _fma(r, C5, C4), _fma(r2, _fma(r, C3, C2), tail + r))
    if not special:
        s = _dbl(sbits)
        return _fma(s, tmp, s)
    if ki & 0x80000000 == 0:
        s = _dbl(sbits - (1009 << 52))
        return 2.0 ** 1009 * _fma(s, tmp, s)
    s = _dbl(sbits + (1022 << 52))
    y = s + s * tmp
    if y < 1.0:
        lo = s - y + s * tmp
        hi = 1.0 + y
        lo = 1.0 - hi + y + lo
        y = (hi + lo) - 1.0
    return 2.0 ** -1022 * y


def test_restatement_matches_host_libm():
    g = np.random.default_rng(99)
    pts = list(-g.uniform(0.0, 746.0, 12000)) + list(-g.uniform(708.0, 746.0, 4000))  # incl. subnormal results
    pts += list(-g.uniform(512.0, 708.0, 2000)) + list(g.uniform(0.0, 709.0, 1000))
    pts += [0.0, -0.0, 1e-300, -1e-300, -745.1332191019412, -745.13321910194122, -708.3964185322641, -1.0]
    for k in g.integers(-95500, 0, 600):  # x * 128 / ln2 next to k + 1/2: the rounding of k
        c = (float(k) + 0.5) / INV
        for d in (-2, -1, 0, 1, 2):
            pts.append(float(np.nextafter(c, math.copysign(math.inf, d))) if d else c)
    bad = [(x, _exp(x), math.exp(x)) for x in pts if -746.0 <= x <= 709.0 and _exp(x) != math.exp(x)]
    assert not bad, f"{len(bad)} of {len(pts)} differ, e.g. {bad[:3]}"
