"""A stack of MoE blocks (BASELINE config 5's shape: gate/up IQ3_S, down Q4_K, shared expert Q8_0, H 2048, F 512,
512 experts, top-10, each layer with its own router and Zipf(1.1) bias) against the CPU oracle, through the C ABI.

Attention and DeltaNet are omitted, as in config 5; a residual x <- x + y (numpy, fp32, the same on both sides) links
the layers so that each layer's routing depends on the previous layers' outputs. The layers' experts are device copies
of layer 0's (moe_copy_experts), so the oracle's view of every layer is layer 0's experts with that layer's router.
Decode (T = 1, the decode kernel) and prefill (two chunks of 2048 tokens, the prefill kernels) are checked, the
prefill on a sample of tokens of both chunks (a token's output depends on that token alone).
"""
import sys

import numpy as np
import pytest

from tests import harness as h
from tests.harness import moe

pytestmark = pytest.mark.gpu
NL = 4
Q8, Q4, I3 = moe.QT_Q8_0, moe.QT_Q4_K, moe.QT_IQ3_S


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def stack():
    say("stack: drawing", NL, "layers")
    L0 = h.Layer(2048, 512, 512, 10, I3, Q4, Q8, Q8, seed=2026, zipf=1.1, nthreads=0)
    blk = L0.block(n_layer=NL, max_tokens=2048, exact_router=True)  # the oracle's bits through every layer
    L0.upload(blk, 0)
    layers = [L0]
    for l in range(1, NL):
        Ll = h.Layer(2048, 512, 512, 10, I3, Q4, Q8, Q8, seed=2026, layer=l, zipf=1.1, experts=[], has_shared=False)
        blk.load_router(l, Ll.router, Ll.bias)
        blk.copy_experts(0, l)
        Ll.experts, Ll.shared, Ll.has_shared = L0.experts, L0.shared, True
        layers.append(Ll)
    yield blk, layers
    blk.close()


def run_oracle(layers, x):
    ids_all = []
    for L in layers:
        y, ids, _ = L.oracle_forward(x, nthreads=16)
        ids_all.append(ids)
        x = x + y
    return x, ids_all


def test_stack_decode(stack):
    blk, layers = stack
    for t in range(3):
        say("stack decode, token", t)
        x = h.tokens(500 + t, 1, 2048)
        xg = x.copy()
        ids_g = []
        for l in range(NL):
            y, ids, _ = blk.forward(l, xg)
            ids_g.append(ids)
            xg = xg + y
        xo, ids_o = run_oracle(layers, x)
        for l in range(NL):
            assert np.array_equal(ids_g[l], ids_o[l]), "layer %d ids" % l
        assert np.array_equal(xg, xo), (h.max_abs(xg, xo), h.rel_l2(xg, xo))
        assert len({tuple(i.ravel()) for i in ids_g}) == NL  # every layer routes differently


def test_stack_prefill_two_chunks(stack):
    blk, layers = stack
    T, chunk = 4096, 2048
    x = h.tokens(4096, T, 2048)
    outs = []
    for c0 in range(0, T, chunk):
        say("stack prefill, chunk at", c0)
        xg = x[c0:c0 + chunk].copy()
        for l in range(NL):
            y, _, _ = blk.forward(l, xg)
            xg = xg + y
        outs.append(xg)
    xg = np.concatenate(outs)
    sample = np.r_[0:12, chunk - 4:chunk + 12, T - 12:T]
    say("stack prefill: oracle on", len(sample), "tokens")
    xo, _ = run_oracle(layers, x[sample])
    assert np.array_equal(xg[sample], xo), (h.max_abs(xg[sample], xo), h.rel_l2(xg[sample], xo))
