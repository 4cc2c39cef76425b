"""The constant tables the kernels carry, recomputed from what fixes them.

  - expf's table (c0ven_amd/csrc/device_math.h): entry i holds the bits of the double nearest 2^(i/32), minus
    i << 47; recomputed with exact rational arithmetic (the nearest double to an irrational is well defined: 2^(i/32)
    is bracketed to 80 bits by integer square roots).
  - the IQ3_S grid (c0ven_amd/csrc/iq3s_grid.h): the sha256 of the 512 u32 words the reference records
    (docs/spec/QUANT_FORMATS.md:546), and equal to the oracle's grid (built from the lattice in oracle/).
"""
import hashlib
import math
import os
import re
from fractions import Fraction

import numpy as np

from tests import harness as h

CSRC = os.path.join(h.ROOT, "c0ven_amd", "csrc")


def macro_values(path, name):
    text = open(path).read()
    m = re.search(r"#define %s\s*\\\n((?:.*\\\n)*.*)\n" % name, text)
    body = m.group(1).replace("\\", " ")
    return [int(v.strip().rstrip("uUlL"), 0) for v in body.split(",") if v.strip()]


def nearest_double_pow2(i):
    """The double nearest 2^(i/32), 1 <= value < 2, as its 64-bit pattern."""
    # 2^(i/32) * 2^K = isqrt^5(2^i * 2^(32K)): the 32nd root by five square roots of a huge integer.
    K = 120
    v = 2 ** i * 2 ** (32 * K)
    for _ in range(5):
        v = math.isqrt(v)
    lo = Fraction(v, 2 ** K)  # within a few 2^-120 of the true value, below it
    m = lo * 2 ** 52          # the value is in [1, 2): mantissa units of 2^-52
    f = math.floor(m)
    frac = m - f
    assert abs(frac - Fraction(1, 2)) > Fraction(1, 2 ** 60)  # not near a tie: rounding is decided
    mant = f + (1 if frac > Fraction(1, 2) else 0)
    return (1023 << 52) + (mant - 2 ** 52) if mant < 2 ** 53 else (1024 << 52)


def test_exp2_table():
    tab = macro_values(os.path.join(CSRC, "device_math.h"), "C0VEN_EXP2_TAB_VALUES")
    assert len(tab) == 32
    for i, t in enumerate(tab):
        assert (t + (i << 47)) % 2 ** 64 == nearest_double_pow2(i), i
    # and the stored value is that double: 2^(i/32) to within half an ulp
    for i, t in enumerate(tab):
        d = np.array([(t + (i << 47)) % 2 ** 64], dtype=np.uint64).view(np.float64)[0]
        assert abs(d - 2 ** (i / 32)) <= 2 ** -52


def test_iq3s_grid_table():
    g = np.array(macro_values(os.path.join(CSRC, "iq3s_grid.h"), "C0VEN_IQ3S_GRID_VALUES"), dtype=np.uint32)
    assert len(g) == 512
    assert hashlib.sha256(g.astype("<u4").tobytes()).hexdigest() == (
        "bd1af4945a1717c65610b0284e4628b9a1ba3b306fae3a06f6e5f597356e349f")
    assert np.array_equal(g, h.orc_grid())
