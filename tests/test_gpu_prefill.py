"""The prefill path (more than 16 tokens: router GEMM, counting-sort dispatch, grouped int8-MFMA GEMMs, combine)
against the CPU oracle, through the C ABI, on the GPU.

With the exact router (MOE_FLAG_EXACT_ROUTER) it reproduces the oracle's every rounding, so ids, weights and y are
held to bit equality; with the default matrix-core router the ids are still the oracle's (its top k are certified, and
summed exactly where the bound leaves them open) and w, y are held to the bar (max-abs 1e-3, rel-L2 1e-4; w 2e-5). The dispatch is checked against a stable counting sort in numpy: the
MoeTiles (shared/moe_tile.h:11-18) cover each expert's assignments in token order, at most MOE_TILE rows a tile.
At BASELINE's config 4 size (2048 tokens, 512 experts, top-10) the oracle runs on a sample of the tokens, since each
token's output depends on that token alone.
"""
import sys

import numpy as np
import pytest

from tests import harness as h
from tests.harness import moe

pytestmark = pytest.mark.gpu
Q8, Q4, I3 = moe.QT_Q8_0, moe.QT_Q4_K, moe.QT_IQ3_S


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def expected_dispatch(ids, E):
    flat = ids.ravel()
    perm, tiles = [], []
    for e in range(E):
        a = np.nonzero(flat == e)[0]
        for i in range(0, len(a), 64):
            tiles.append((e, e, len(perm) + i, min(64, len(a) - i)))
        perm.extend(a.tolist())
    return np.array(tiles, dtype=np.uint32).reshape(-1, 4), np.array(perm, dtype=np.uint32)


def check_exact(y, ids, w, yo, io, wo, exact=True):
    h.check_block(y, ids, w, yo, io, wo, exact)


ROUTERS = [False, True]  # the default (matrix-core, certified) router, then the exact one
@pytest.mark.parametrize("types", [(Q8, Q8, Q8, Q8), (Q4, Q4, Q4, Q4), (I3, I3, I3, I3), (I3, Q4, Q8, Q8),
                                   (Q4, Q8, I3, Q4)])
@pytest.mark.parametrize("T", [17, 100, 300])
@pytest.mark.parametrize("exact", ROUTERS)
def test_prefill_small(types, T, exact):
    gt, dt, sgt, sdt = types
    say("prefill small", [moe.TYPE_NAMES[t] for t in types], "T", T, "exact router", exact)
    L = h.Layer(512, 256, 64, 4, gt, dt, sgt, sdt, seed=31 + T, zipf=1.1 if T == 100 else None)
    blk = L.block(max_tokens=512, exact_router=exact)
    L.upload(blk)
    x = h.tokens(5 + T, T, 512)
    y, ids, w = blk.forward(0, x)
    tiles, perm = blk.prefill_dispatch(T)
    et, ep = expected_dispatch(ids, L.E)
    assert np.array_equal(tiles, et) and np.array_equal(perm, ep)
    check_exact(y, ids, w, *L.oracle_forward(x), exact)
    blk.close()


@pytest.mark.parametrize("H,F", [(1024, 512), (2048, 256)])
def test_prefill_shapes_no_shared_and_limit(H, F):
    say("prefill shapes", H, F)
    L = h.Layer(H, F, 32, 8, Q4, I3, has_shared=False, seed=9, swiglu_limit=0.02)
    blk = L.block(max_tokens=256)
    L.upload(blk)
    x = h.tokens(3, 130, H)
    y, ids, w = blk.forward(0, x)
    check_exact(y, ids, w, *L.oracle_forward(x), blk.bit_exact(len(x)))
    blk.close()


@pytest.mark.parametrize("H,F,types", [(2560, 640, (Q4, Q8, Q4, Q8)), (2560, 640, (I3, Q8, I3, Q8)),
                                         (1536, 256, (Q4, Q4, I3, Q4))])
def test_prefill_unit_counts(H, F, types):
    # The Q4_K and IQ3_S gate/up kernels run their unit loop for U - 1 units and then the last one apart (whether a
    # next unit's loads are issued is a compile-time flag): U = 10 and 6 here, besides 2, 4 and 8 above.
    gt, dt, sgt, sdt = types
    say("prefill unit counts", H, F, [moe.TYPE_NAMES[t] for t in types])
    L = h.Layer(H, F, 32, 6, gt, dt, sgt, sdt, seed=77 + H)
    blk = L.block(max_tokens=256)
    L.upload(blk)
    x = h.tokens(11, 150, H)
    y, ids, w = blk.forward(0, x)
    check_exact(y, ids, w, *L.oracle_forward(x), blk.bit_exact(len(x)))
    blk.close()


@pytest.mark.parametrize("exact", ROUTERS)
def test_prefill_extreme_block_sums(exact):
    """Tokens whose q8_K codes are all +-127 (constant rows of either sign, and rows whose 32-value blocks alternate
    in sign) give block sums of +-4064, the ends of the split 64 hi + lo the Q4_K minimum term's f16 operand holds
    (hi -64 and 63); with random rows between them. Q4_K everywhere, so every GEMM takes that path."""
    say("prefill extreme block sums, exact router", exact)
    H = 1024
    L = h.Layer(H, 256, 64, 6, Q4, Q4, Q4, Q4, seed=404)
    blk = L.block(max_tokens=128, exact_router=exact)
    L.upload(blk)
    x = h.tokens(41, 96, H).copy()
    sign = np.where((np.arange(H) // 32) % 2 == 0, 1.0, -1.0).astype(np.float32)
    for t in range(0, 96, 4):
        x[t] = 0.75 + 0.01 * t
        x[t + 1] = -(0.5 + 0.01 * t)
        x[t + 2] = sign * (0.25 + 0.01 * t)
    y, ids, w = blk.forward(0, x)
    check_exact(y, ids, w, *L.oracle_forward(x), exact)
    blk.close()


def test_prefill_then_decode_share_a_context():
    """Both paths on one context, alternating: each call's result stands alone."""
    say("prefill and decode alternate")
    L = h.Layer(512, 256, 64, 6, Q4, Q8, seed=77)
    blk = L.block(max_tokens=128)
    L.upload(blk)
    for T in (40, 3, 128, 16, 17):
        x = h.tokens(T, T, 512)
        y, ids, w = blk.forward(0, x)
        check_exact(y, ids, w, *L.oracle_forward(x), blk.bit_exact(len(x)))
    blk.close()


def test_prefill_forwards_in_a_row():
    """Prefill forwards of different lengths on one context: each clears the dispatch masks its routing sets (a shorter
    forward leaves an earlier one's bits in windows it does not read), so tiles, perm and y stand alone."""
    say("prefill forwards in a row")
    L = h.Layer(512, 256, 64, 6, Q4, Q4, seed=123, zipf=1.1)
    blk = L.block(max_tokens=320)
    L.upload(blk)
    for i, T in enumerate((300, 17, 300, 130)):
        x = h.tokens(200 + i, T, 512)
        y, ids, w = blk.forward(0, x)
        tiles, perm = blk.prefill_dispatch(T)
        et, ep = expected_dispatch(ids, L.E)
        assert np.array_equal(tiles, et) and np.array_equal(perm, ep), T
        check_exact(y, ids, w, *L.oracle_forward(x), blk.bit_exact(len(x)))
    blk.close()


@pytest.mark.parametrize("exact", ROUTERS)
def test_prefill_config4_sampled(exact):
    """2048 tokens, H 2048, F 512, 512 experts, top-10 + shared, Q4_K, Zipf(1.1)."""
    say("prefill config 4, exact router", exact)
    L = h.Layer(2048, 512, 512, 10, Q4, Q4, seed=2026, zipf=1.1, nthreads=0)
    blk = L.block(max_tokens=2048, exact_router=exact)
    L.upload(blk)
    T = 2048
    x = h.tokens(2026, T, 2048)
    y, ids, w = blk.forward(0, x)
    tiles, perm = blk.prefill_dispatch(T)
    et, ep = expected_dispatch(ids, L.E)
    assert np.array_equal(tiles, et) and np.array_equal(perm, ep)
    assert tiles[:, 3].sum() == T * 10 and tiles[:, 3].max() <= 64
    _, io, wo = L.oracle_route(x)
    assert np.array_equal(ids, io) and (np.array_equal(w, wo) if exact else h.max_abs(w, wo) <= h.W_TOL)
    if not exact:
        say("tokens whose top k were summed exactly:", blk.prefill_exact_tokens())
    sample = np.r_[0:48, 1000:1016, T - 48:T]
    yo, io2, wo2 = L.oracle_forward(x[sample], nthreads=16)
    assert np.array_equal(io2, ids[sample])
    check_exact(y[sample], ids[sample], w[sample], yo, io2, wo2, exact)
    blk.close()


def test_prefill_dispatch_many_windows():
    """A long prefill (T k > 40960; 66 windows of 64 tokens, more than the 32 masks a dispatch thread loads at once,
    so its count runs over several batches of windows). Tiles and perm against the stable counting sort; ids, w and
    y against the oracle on a sample."""
    say("prefill dispatch, 4200 tokens x k 10")
    L = h.Layer(512, 256, 64, 10, Q4, Q8, seed=4200, zipf=1.1)
    T = 4200
    blk = L.block(max_tokens=T)
    L.upload(blk)
    x = h.tokens(4200, T, 512)
    y, ids, w = blk.forward(0, x)
    tiles, perm = blk.prefill_dispatch(T)
    et, ep = expected_dispatch(ids, L.E)
    assert T * 10 > 40960
    assert np.array_equal(tiles, et) and np.array_equal(perm, ep)
    _, io, wo = L.oracle_route(x)
    assert np.array_equal(ids, io) and h.max_abs(w, wo) <= h.W_TOL
    sample = np.r_[0:40, 2090:2110, T - 40:T]
    yo, io2, wo2 = L.oracle_forward(x[sample], nthreads=16)
    check_exact(y[sample], ids[sample], w[sample], yo, io2, wo2, False)
    blk.close()


def test_prefill_config5_chunk_sampled():
    """BASELINE config 5's layer at full size, one 2048-token prefill chunk: H 2048, F 512, 512 experts, top-10,
    gate/up IQ3_S, down Q4_K, shared expert Q8_0, Zipf(1.1). Hot experts span many 64-row tiles. ids and w on every
    token, y on a sample (each token's y depends on that token alone)."""
    say("prefill config 5 chunk")
    L = h.Layer(2048, 512, 512, 10, I3, Q4, Q8, Q8, seed=2026, zipf=1.1, nthreads=0)
    blk = L.block(max_tokens=2048)
    L.upload(blk)
    T = 2048
    x = h.tokens(2027, T, 2048)
    y, ids, w = blk.forward(0, x)
    tiles, perm = blk.prefill_dispatch(T)
    et, ep = expected_dispatch(ids, L.E)
    assert np.array_equal(tiles, et) and np.array_equal(perm, ep)
    assert tiles[:, 3].sum() == T * 10 and np.bincount(tiles[:, 0]).max() >= 8  # a hot expert over >= 8 tiles
    _, io, wo = L.oracle_route(x)
    assert np.array_equal(ids, io) and h.max_abs(w, wo) <= h.W_TOL
    sample = np.r_[0:32, 1024:1040, T - 32:T]
    yo, io2, wo2 = L.oracle_forward(x[sample], nthreads=16)
    check_exact(y[sample], ids[sample], w[sample], yo, io2, wo2, False)
    blk.close()
