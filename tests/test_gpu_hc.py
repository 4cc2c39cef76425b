"""moe_forward_hc: the block with its hyper-connection mix and combine fused into the decode launch (MODEL_LAYER.md
1.1-1.2; model.cpp:1350-1416 runs them as separate kernels) against the oracle's mix, block and combine, bit for bit:
the updated streams R, y, the routing."""
import sys

import numpy as np
import pytest

from tests import harness as h
from tests.harness import moe

pytestmark = pytest.mark.gpu


def say(*a):
    print("[hc]", *a, flush=True)
    sys.stdout.flush()


@pytest.mark.parametrize("shape", [(512, 256, 32, 4, 64), (2560, 640, 64, 8, 320)])
@pytest.mark.parametrize("types", [(moe.QT_Q4_K, moe.QT_Q8_0, moe.QT_Q8_0, moe.QT_Q8_0),
                                   (moe.QT_IQ3_XXS, moe.QT_IQ4_NL, moe.QT_Q4_K, moe.QT_IQ4_NL)])
def test_forward_hc(shape, types):
    H, F, E, K, lr = shape
    gt, dt, sgt, sdt = types
    if H % 256 or (dt == moe.QT_Q4_K and F % 256):
        pytest.skip("shape not of these types")
    say("forward_hc", shape, [moe.TYPE_NAMES[t] for t in types])
    L = h.Layer(H, F, E, K, gt, dt, sgt, sdt, seed=H + lr, zipf=1.1)
    hc = h.HcModule(H, lr, seed=11)
    blk = moe.MoeBlock(H, F, E, K, gt, dt, True, sgt, sdt, n_layer=2, max_tokens=16, hc_lr=lr)
    L.upload(blk, 1)
    hc.load(blk, 1)
    r = np.random.default_rng(H)
    for T in (1, 8, 16):
        R = r.standard_normal((T, 4, H)).astype(np.float32)
        R2, y, ids, w = blk.forward_hc(1, R)
        x, inj = hc.pre(R)
        yo, io, wo = L.oracle_forward(x)
        Ro = h.HcModule.post(R, inj, yo)
        assert np.array_equal(ids, io) and np.array_equal(w, wo), T
        assert np.array_equal(y, yo), (T, h.max_abs(y, yo))
        assert np.array_equal(R2, Ro), (T, h.max_abs(R2, Ro))
        # The plain forward on the oracle's x gives the same y (the mix is the only difference).
        y2, _, _ = blk.forward(1, x)
        assert np.array_equal(y2, yo)
    blk.close()


def test_forward_hc_requires_module():
    blk = moe.MoeBlock(512, 256, 8, 2, moe.QT_Q8_0, moe.QT_Q8_0, hc_lr=64)
    L = h.Layer(512, 256, 8, 2, moe.QT_Q8_0, moe.QT_Q8_0, seed=4)
    L.upload(blk)
    with pytest.raises(moe.MoeError):  # no moe_load_hc yet
        blk.forward_hc(0, np.zeros((1, 4, 512), np.float32))
    blk.close()
    with pytest.raises(moe.MoeError):  # hc_lr not a multiple of 8
        moe.MoeBlock(512, 256, 8, 2, moe.QT_Q8_0, moe.QT_Q8_0, hc_lr=100)


@pytest.mark.parametrize("shape", [(512, 256, 32, 4, 64), (2560, 640, 64, 8, 320)])
@pytest.mark.parametrize("fixed_order", [False, True])
def test_forward_hc_prefill(shape, fixed_order):
    """More tokens than the decode kernel takes: the mix's kernels (fp64 matrix cores within a bound, the open sums in
    the fixed order; with hc_fixed_order every down sum in the fixed order), the prefill block, the combine's kernel;
    R, y and the routing against the oracle's, bit for bit (the exact router: the oracle's weights and y)."""
    H, F, E, K, lr = shape
    say("forward_hc prefill", shape, "fixed order" if fixed_order else "bound")
    L = h.Layer(H, F, E, K, moe.QT_Q4_K, moe.QT_Q8_0, moe.QT_Q8_0, moe.QT_Q8_0, seed=H + lr + 1, zipf=1.1)
    hc = h.HcModule(H, lr, seed=12)
    blk = moe.MoeBlock(H, F, E, K, moe.QT_Q4_K, moe.QT_Q8_0, True, moe.QT_Q8_0, moe.QT_Q8_0, n_layer=1,
                       max_tokens=320, hc_lr=lr, exact_router=True, hc_fixed_order=fixed_order)
    L.upload(blk, 0)
    hc.load(blk, 0)
    r = np.random.default_rng(H + 7)
    for T in ((17, 100) if fixed_order else (17, 100, 320)):
        R = r.standard_normal((T, 4, H)).astype(np.float32)
        R2, y, ids, w = blk.forward_hc(0, R)
        x, inj = hc.pre(R)
        yo, io, wo = L.oracle_forward(x)
        Ro = h.HcModule.post(R, inj, yo)
        assert np.array_equal(ids, io) and np.array_equal(w, wo), T
        assert np.array_equal(y, yo), (T, h.max_abs(y, yo))
        assert np.array_equal(R2, Ro), (T, h.max_abs(R2, Ro))
    blk.close()
