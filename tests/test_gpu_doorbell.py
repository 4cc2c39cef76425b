"""The CPU/GPU hybrid (core/models/qwen4exp/layout.h:64-71 MissJob, layer.cl:838-884, model.cpp:1597-1627): a layer
whose routed experts are partly off the device. The decode kernel computes the resident ones, publishes each token's
misses in its record in host memory (the step number last), and its combine waits for the host's answer. Here the host
side is the test: it polls the records, answers with the oracle's compute_many over the misses (the role
CpuExperts::compute_many plays in the reference), and stores the step. The block's output is checked bit for bit
against the oracle's hybrid sum (resident experts in rank order, + gs s, + the misses' sum).

Also: the other launch-shape guarantees of the persistent decode kernel (a grid of any multiple of 8, larger than the
device holds at once; a decode launched while another stream's prefill kernels occupy the device)."""
import ctypes as C
import sys
import time

import numpy as np
import pytest

from tests import harness as h
from tests.harness import moe

pytestmark = pytest.mark.gpu
JOB_WORDS = 2 + 3 * 16  # seq, nmiss, ids[16], w[16], all[16]; then x


def say(*a):
    print("[doorbell]", *a, flush=True)
    sys.stdout.flush()


def oracle_resident(L, resident, x):
    Lo, keep = L._orc_layer()
    y = np.empty((x.shape[0], L.H), dtype=np.float32)
    r = np.ascontiguousarray(resident, dtype=np.uint8)
    assert h.oracle.orc_moe_forward_resident(C.byref(Lo), h.ptr(r), h.ptr(x), x.shape[0], L.H, h.ptr(y), L.H, 8) == 0
    del keep
    return y


def answer(L, blk, T, step, timeout=10.0):
    """The host side: wait for every token's record of this step, answer the misses, store the step."""
    jobs, stride, ans_y, ans_seq = blk.miss_buffers()
    H = L.H
    rec = lambda t: np.ctypeslib.as_array((C.c_uint8 * stride).from_address(jobs + t * stride))
    ans = np.ctypeslib.as_array((C.c_float * (16 * H)).from_address(ans_y)).reshape(16, H)
    seq = np.ctypeslib.as_array((C.c_uint32 * 1).from_address(ans_seq))
    t0 = time.time()
    cpu_jobs, xs, nmiss = [], np.zeros((T, H), np.float32), []
    for t in range(T):
        r = rec(t)
        while r[:4].view(np.uint32)[0] != step:
            assert time.time() - t0 < timeout, "token %d's record did not arrive" % t
        words = r[:4 * JOB_WORDS].view(np.uint32)
        n = int(words[1])
        ids = words[2:2 + 16].view(np.int32)[:n]
        w = words[18:18 + 16].view(np.float32)[:n]
        nmiss.append(n)
        if n:
            xs[t] = r[4 * JOB_WORDS:4 * JOB_WORDS + 4 * H].view(np.float32)
            cpu_jobs += [(L.experts[int(e)], t, float(wk)) for e, wk in zip(ids, w)]
    if cpu_jobs:
        y = h.orc_compute_many(L.gate_type, L.down_type, L.H, L.F, cpu_jobs, xs)
        ans[:T] = y
        seq[0] = step  # after the answer (x86 keeps the stores in order)
    return nmiss, xs


@pytest.mark.parametrize("T", [1, 8])
def test_misses_answered_by_the_host(T):
    L = h.Layer(512, 256, 64, 8, moe.QT_Q4_K, moe.QT_Q8_0, seed=71 + T, zipf=1.1)
    blk = L.block()
    L.upload(blk)
    resident = np.ones(L.E, np.uint8)
    resident[::3] = 0  # a third of the experts off the device
    blk.set_resident(0, resident)
    blk.miss_buffers()
    dev = h.Dev()
    for rep in range(3):  # consecutive steps: each answer belongs to its own step
        say("T", T, "step", rep)
        x = h.tokens(700 + 10 * T + rep, T, 512)
        xd, yd = dev.put(x), dev.alloc(T * 512 * 4)
        idd, wd = dev.alloc(T * 8 * 4), dev.alloc(T * 8 * 4)
        blk.forward_async(0, xd, T, yd, idd, wd)
        nmiss, xs = answer(L, blk, T, blk.last_step())
        blk.check()
        y, ids = dev.get(yd, (T, 512), np.float32), dev.get(idd, (T, 8), np.int32)
        _, io, _ = L.oracle_route(x)
        assert np.array_equal(ids, io)
        assert nmiss == [int((resident[io[t]] == 0).sum()) for t in range(T)]
        for t in range(T):
            if nmiss[t]:
                assert np.array_equal(xs[t], x[t])  # the record carries the token's input
        yo = oracle_resident(L, resident, x)
        assert np.array_equal(y, yo), (h.max_abs(y, yo), h.rel_l2(y, yo))
    assert sum(nmiss) > 0
    with pytest.raises(moe.MoeError):  # the prefill path takes only fully resident layers
        blk2 = L.block(max_tokens=64)
        L.upload(blk2)
        blk2.set_resident(0, resident)
        blk2.forward(0, h.tokens(1, 40, 512))
    blk.set_resident(0, None)  # all resident again: no records to answer
    x = h.tokens(799, T, 512)
    y, ids, w = blk.forward(0, x)
    h.check_block(y, ids, w, *L.oracle_forward(x))
    dev.free()
    blk.close()


@pytest.mark.parametrize("grid", [8, "2x", "4x"])
def test_decode_any_grid(grid):
    """A grid of 8 work-groups, or two or four times what the device holds at once (the work-groups past the first
    wave start only as others exit): the same bits."""
    L = h.Layer(512, 256, 64, 8, moe.QT_Q4_K, moe.QT_Q8_0, seed=61, zipf=1.1)
    blk = L.block()
    L.upload(blk)
    g = {"2x": 2, "4x": 4}[grid] * moe.lib.moe_grid(blk.h) if isinstance(grid, str) else grid
    say("decode grid", g)
    assert moe.lib.moe_set_grid(blk.h, g) == moe.MOE_OK
    for T in (1, 8, 16):
        x = h.tokens(610 + T, T, 512)
        y, ids, w = blk.forward(0, x)  # raises MoeError(MOE_TIMEOUT) if a wait gave up
        h.check_block(y, ids, w, *L.oracle_forward(x))
    assert moe.lib.moe_set_grid(blk.h, 7) == moe.MOE_BAD_ARGUMENT
    assert moe.lib.moe_set_grid(blk.h, 0) == moe.MOE_OK
    blk.close()


def test_decode_beside_another_streams_kernels():
    """A decode forward enqueued while another context's prefill kernels (on that context's stream) hold the device:
    the decode kernel's work-groups start as the device frees up, and its result is the oracle's."""
    Lb = h.Layer(2048, 512, 128, 8, moe.QT_Q4_K, moe.QT_Q4_K, seed=62)
    big = Lb.block(max_tokens=2048)
    Lb.upload(big)
    L = h.Layer(512, 256, 64, 8, moe.QT_Q4_K, moe.QT_Q8_0, seed=63, zipf=1.1)
    blk = L.block()
    L.upload(blk)
    dev = h.Dev()
    xb = h.tokens(64, 2048, 2048)
    xbd, ybd = dev.put(xb), dev.alloc(xb.nbytes)
    for T in (1, 8):
        say("decode beside prefill, T", T)
        for _ in range(4):
            big.forward_async(0, xbd, 2048, ybd)
        x = h.tokens(620 + T, T, 512)
        y, ids, w = blk.forward(0, x)
        h.check_block(y, ids, w, *L.oracle_forward(x))
        big.check()
    dev.free()
    big.close()
    blk.close()
