"""moe_forward_async_noalloc (the decode entry point that allocates nothing: its scratch is a static per-GPU array)
against moe_forward_async on the same inputs, through the C ABI: ids, w and y bit-equal, on consecutive calls (the
second with fewer tokens, so stale records of the first must not be read), across two contexts sharing the GPU's
array, and the refusals (too many tokens; a shape whose scratch exceeds the array).
"""
import ctypes as C

import numpy as np
import pytest

from tests import harness as h
from tests.harness import moe

pytestmark = pytest.mark.gpu


Dev = h.Dev


def run(blk, dev, fn, x, layer=0):
    T, H = x.shape
    K = blk.cfg.n_used
    xd, yd, idd, wd = dev.put(x), dev.alloc(T * H * 4), dev.alloc(T * K * 4), dev.alloc(T * K * 4)
    fn(layer, xd, T, yd, idd, wd)
    blk.check()
    return dev.get(yd, (T, H), np.float32), dev.get(idd, (T, K), np.int32), dev.get(wd, (T, K), np.float32)


def same(a, b):
    for u, v in zip(a, b):
        assert np.array_equal(u, v)


def test_noalloc_equals_forward_async():
    dev = Dev()
    La = h.Layer(512, 256, 64, 6, moe.QT_Q4_K, moe.QT_Q8_0, seed=11, zipf=1.1)
    Lb = h.Layer(1024, 512, 32, 4, moe.QT_IQ3_S, moe.QT_Q4_K, moe.QT_Q8_0, moe.QT_Q8_0, seed=12)
    a, b = La.block(), Lb.block()
    La.upload(a)
    Lb.upload(b)
    for T, L, blk, seed in ((8, La, a, 1), (3, La, a, 2), (5, Lb, b, 3), (16, La, a, 4), (1, Lb, b, 5), (2, La, a, 6)):
        x = h.tokens(seed, T, L.H)
        ref = run(blk, dev, blk.forward_async, x)
        got = run(blk, dev, blk.forward_async_noalloc, x)
        same(got, ref)
        yo, io, wo = L.oracle_forward(x)
        same(got, (yo, io, wo))
    a.close()
    b.close()
    dev.free()


def test_noalloc_refusals():
    dev = Dev()
    L = h.Layer(512, 256, 16, 2, moe.QT_Q8_0, moe.QT_Q8_0, seed=13)
    blk = L.block(max_tokens=64)
    L.upload(blk)
    x = h.tokens(1, 17, 512)
    xd, yd = dev.put(x), dev.alloc(x.nbytes)
    with pytest.raises(moe.MoeError) as e:
        blk.forward_async_noalloc(0, xd, 17, yd)
    assert e.value.status == moe._lib.MOE_BAD_ARGUMENT
    blk.close()
    big = moe.MoeBlock(8192, 8192, 16, 16, moe.QT_Q8_0, moe.QT_Q8_0, has_shared=False, max_tokens=16)
    xb = np.zeros((1, 8192), np.float32)
    xd2, yd2 = dev.put(xb), dev.alloc(xb.nbytes)
    with pytest.raises(moe.MoeError) as e:
        big.forward_async_noalloc(0, xd2, 1, yd2)
    assert e.value.status == moe._lib.MOE_BAD_ARGUMENT and "exceeds" in str(e.value)
    big.close()
    dev.free()
