"""The CPU baseline (oracle/cpu_fast.c) against the oracle: the same bits (ids, weights and y bit-equal) for every
weight type and type mix, with and without the shared expert and the swiglu limit. This is what lets bench.py report
it as the reference CPU path's timing: it computes exactly what the oracle computes."""
import ctypes as C

import numpy as np
import pytest

from tests import harness as h
from tests.harness import moe

Q8, Q4, I3 = moe.QT_Q8_0, moe.QT_Q4_K, moe.QT_IQ3_S
o = h.oracle
o.orc_fast_moe_forward.restype = C.c_int
o.orc_fast_moe_forward.argtypes = o.orc_moe_forward.argtypes
o.orc_fast_isa.restype = C.c_char_p


@pytest.mark.parametrize("types,shared,limit", [((Q8, Q8, Q8, Q8), True, 0.0), ((Q4, Q4, Q4, Q4), True, 0.0),
                                                ((I3, I3, I3, I3), True, 0.0), ((I3, Q4, Q8, Q8), True, 0.0),
                                                ((Q4, I3, Q4, Q8), False, 0.02)])
def test_fast_equals_oracle(types, shared, limit):
    L = h.Layer(512, 256, 32, 4, *types, has_shared=shared, seed=71, zipf=1.1, swiglu_limit=limit)
    x = h.tokens(9, 37, 512)
    yo, io, wo = L.oracle_forward(x)
    y, ids, w = h.fast_forward(L, x, nthreads=4)
    assert np.array_equal(ids, io) and np.array_equal(w, wo)
    assert np.array_equal(y, yo), (h.max_abs(y, yo), o.orc_fast_isa().decode())
