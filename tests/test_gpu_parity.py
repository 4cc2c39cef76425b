"""The HIP path against the CPU oracle, through the C ABI (libc0ven_moe.so), on the GPU.

The bar (north_star): top-k expert ids and decoded weight blocks bit-exact; the block's output within max-abs 1e-3
and rel-L2 1e-4. The decode path reproduces the oracle's every rounding (its ORACLE ORDER, libm's expf), so these
tests also hold its output to bit equality, and report the distance when it is not.
"""
import sys

import numpy as np
import pytest

from tests import harness as h
from tests.harness import moe

pytestmark = pytest.mark.gpu
rng = np.random.default_rng(7)
TOL_ABS, TOL_REL = 1e-3, 1e-4


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def check_block(y, ids, w, yo, io, wo, exact=True):
    h.check_block(y, ids, w, yo, io, wo, exact)


def random_blocks(qtype, nblocks):
    nv, nb = moe.BLOCK[qtype]
    b = rng.integers(0, 256, size=(nblocks, nb), dtype=np.uint8)
    reach = {moe.QT_Q8_0: [(0, 128)], moe.QT_Q4_K: [(0, 63 * 15), (2, 63)], moe.QT_IQ3_S: [(0, 31 * 15)],
             moe.QT_IQ4_NL: [(0, 127)], moe.QT_Q2_0: [(0, 2)], moe.QT_IQ3_XXS: [(0, 62 * 31)],
             moe.QT_IQ2_S: [(0, 43 * 31)], moe.QT_Q5_K: [(0, 63 * 31), (2, 63)], moe.QT_Q6_K: [(208, 127 * 32)],
             moe.QT_IQ4_XS: [(0, 31 * 127)]}[qtype]
    for k in range(nblocks):
        for off, r in reach:
            v = np.ldexp(1.0 + rng.integers(0, 1024) / 1024.0, int(rng.integers(0, 3)) - 5) / r
            b[k, off:off + 2] = np.frombuffer(np.float16(v).tobytes(), np.uint8)
    return b.ravel()


@pytest.fixture(scope="module")
def tiny_block():
    blk = moe.MoeBlock(512, 256, 8, 2, moe.QT_Q8_0, moe.QT_Q8_0)
    blk.set_codebooks(h.CODEBOOKS)
    yield blk
    blk.close()


@pytest.mark.parametrize("qtype", [moe.QT_Q8_0, moe.QT_Q4_K, moe.QT_IQ3_S, moe.QT_IQ4_NL, moe.QT_Q2_0, moe.QT_IQ3_XXS,
                                   moe.QT_IQ2_S, moe.QT_Q5_K, moe.QT_Q6_K, moe.QT_IQ4_XS])
@pytest.mark.parametrize("rows,cols", [(128, 512), (100, 256)])
def test_dequantize_bit_exact(tiny_block, qtype, rows, cols):
    say("dequantize", moe.TYPE_NAMES[qtype], rows, cols)
    for src in ("random", "quantised"):
        if src == "random":
            m = random_blocks(qtype, rows * cols // moe.BLOCK[qtype][0])
        else:
            m = moe.synth_matrix(3, 1, qtype, rows, cols)
        got = tiny_block.dequantize(qtype, m, rows, cols)
        want = np.stack([h.orc_dequant(qtype, m[r * moe.row_bytes(qtype, cols):(r + 1) * moe.row_bytes(qtype, cols)],
                                       cols) for r in range(rows)])
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), src


SMALL_TYPES = [
    (moe.QT_Q8_0, moe.QT_Q8_0, moe.QT_Q8_0, moe.QT_Q8_0),
    (moe.QT_Q4_K, moe.QT_Q4_K, moe.QT_Q4_K, moe.QT_Q4_K),
    (moe.QT_IQ3_S, moe.QT_IQ3_S, moe.QT_IQ3_S, moe.QT_IQ3_S),
    (moe.QT_IQ3_S, moe.QT_Q4_K, moe.QT_Q8_0, moe.QT_Q8_0),  # config 5's mix
    (moe.QT_Q4_K, moe.QT_Q8_0, moe.QT_IQ3_S, moe.QT_Q4_K),
]


@pytest.mark.parametrize("types", SMALL_TYPES, ids=lambda t: "-".join(moe.TYPE_NAMES[x] for x in t))
def test_forward_small(types):
    gt, dt, sgt, sdt = types
    L = h.Layer(512, 256, 32, 4, gt, dt, sgt, sdt, seed=11, zipf=1.1)
    blk = L.block()
    L.upload(blk)
    for T in (1, 3, 8, 16):
        say("forward_small", [moe.TYPE_NAMES[t] for t in types], "T", T)
        x = h.tokens(100 + T, T, 512)
        y, ids, w = blk.forward(0, x)
        check_block(y, ids, w, *L.oracle_forward(x))
    blk.close()


def test_forward_no_shared_and_swiglu_limit():
    for has_shared, limit in ((False, 0.0), (True, 0.25), (False, 0.1)):
        say("forward no-shared/limit", has_shared, limit)
        L = h.Layer(512, 512, 16, 3, moe.QT_Q4_K, moe.QT_IQ3_S, has_shared=has_shared, seed=5, swiglu_limit=limit,
                    sigma=0.05)
        blk = L.block()
        L.upload(blk)
        x = h.tokens(5, 5, 512)
        y, ids, w = blk.forward(0, x)
        check_block(y, ids, w, *L.oracle_forward(x))
        blk.close()


@pytest.mark.parametrize("tie", ["pairs", "all"])
def test_routing_ties(tie):
    """Exactly equal logits: the lower expert id ranks first (route.h's order). "pairs" makes experts 2i and 2i + 1
    equal; "all" makes every logit of a token equal, so every key is a top-k candidate (K = 16, the most)."""
    L = h.Layer(512, 256, 128, 16, moe.QT_Q8_0, moe.QT_Q8_0, seed=23)
    E = L.E
    if tie == "pairs":
        L.router[1:E:2] = L.router[0:E:2]
    else:
        L.router[:E] = L.router[0]
    blk = L.block(max_tokens=32)
    L.upload(blk)
    for T in (1, 5, 16, 24):  # 24: the prefill path
        say("routing ties", tie, "T", T)
        x = h.tokens(300 + T, T, 512)
        y, ids, w = blk.forward(0, x)
        yo, io, wo = L.oracle_forward(x)
        if tie == "all":
            assert (io == np.arange(16)).all()
        check_block(y, ids, w, yo, io, wo, blk.bit_exact(T))
    if tie == "all":
        assert blk.prefill_exact_tokens() == 24  # every prefill token's top k left open by the bound
    blk.close()


def routed_layer(types, T, seed, zipf, E=512, K=10, H=2048, F=512):
    """A full-size layer with only the experts x routes to drawn (the others stay zero on the device, never read)."""
    gt, dt, sgt, sdt = types
    L = h.Layer(H, F, E, K, gt, dt, sgt, sdt, seed=seed, zipf=zipf, experts=[])
    x = h.tokens(seed, T, H)
    _, ids, _ = L.oracle_route(x)
    for e in sorted(set(ids.ravel().tolist())):
        L.experts[e] = L._expert(e, gt, dt, 0.02, 0)
    return L, x


CONFIGS = [
    ("config1-Q8_0-T1", (moe.QT_Q8_0,) * 4, 1, None),
    ("config2-Q4_K-T8-zipf", (moe.QT_Q4_K,) * 4, 8, 1.1),
    ("config3-IQ3_S-T1", (moe.QT_IQ3_S,) * 4, 1, None),
    ("config3-IQ3_S-T4", (moe.QT_IQ3_S,) * 4, 4, None),
    ("config5-mixed-T1", (moe.QT_IQ3_S, moe.QT_Q4_K, moe.QT_Q8_0, moe.QT_Q8_0), 1, 1.1),
    ("config2-Q4_K-T16-zipf", (moe.QT_Q4_K,) * 4, 16, 1.1),
]


@pytest.mark.parametrize("name,types,T,zipf", CONFIGS, ids=[c[0] for c in CONFIGS])
def test_forward_full_size(name, types, T, zipf):
    say("full size", name)
    L, x = routed_layer(types, T, 17, zipf)
    blk = L.block()
    L.upload(blk)
    y, ids, w = blk.forward(0, x)
    check_block(y, ids, w, *L.oracle_forward(x))
    y2, _, _ = blk.forward(0, x)  # deterministic: the counters reset themselves
    assert np.array_equal(y, y2)
    blk.close()


def test_forward_experts_is_compute_many():
    say("forward_experts")
    H, F, E = 512, 256, 6
    for gt, dt in ((moe.QT_Q4_K, moe.QT_Q8_0), (moe.QT_IQ3_S, moe.QT_IQ3_S)):
        L = h.Layer(H, F, E, 2, gt, dt, seed=21)
        blk = L.block()
        L.upload(blk)
        x = h.tokens(21, 4, H)
        jobs = [(0, 0, 0.5), (1, 0, 0.25), (1, 1, 0.75), (5, 1, 0.125), (1, 2, 1.0), (E, 2, 0.5), (3, 0, -0.5)]
        y = blk.forward_experts([(0, e, t, w) for e, t, w in jobs], x)
        mats = lambda e: L.shared if e == E else L.experts[e]
        yo = h.orc_compute_many(gt, dt, H, F, [(mats(e), t, w) for e, t, w in jobs if e != E], x)
        # the shared expert's job has the shared types; compute_many takes one shape, so sum it in separately
        ys = h.orc_compute_many(L.sh_gate_type, L.sh_down_type, H, F, [(mats(E), 2, 0.5)], x)
        yo[2] = yo[2] + ys[2]  # token 2: its routed job first, then the shared one, as the job order gives
        assert not y[3].any()  # a token without jobs is zero
        assert h.max_abs(y, yo) <= TOL_ABS and h.rel_l2(y, yo) <= TOL_REL
        assert np.array_equal(y, yo)
        blk.close()


def test_bad_arguments_do_not_crash(tiny_block):
    say("bad arguments")
    x = np.zeros((17, 512), np.float32)
    with pytest.raises(moe.MoeError) as e:
        tiny_block.forward(0, x)
    assert e.value.status == 2
    with pytest.raises(moe.MoeError) as e:
        tiny_block.forward(3, x[:1])
    assert e.value.status == 2
    with pytest.raises(moe.MoeError):
        moe.MoeBlock(500, 256, 8, 2, moe.QT_Q8_0, moe.QT_Q8_0)
    # Device buffers must be 16-byte aligned (the kernels read and write them in 8- and 16-byte pieces): refused
    # before anything is enqueued.
    import ctypes
    import bench
    hip = bench.Hip()
    buf = hip.malloc(2 * 512 * 4 + 64)
    base = buf.value
    for xo, yo in ((4, 0), (0, 8)):
        with pytest.raises(moe.MoeError) as e:
            tiny_block.forward_async(0, ctypes.c_void_p(base + xo), 1, ctypes.c_void_p(base + 2048 + 16 + yo))
        assert e.value.status == 2
    hip.sync()
    hip.rt.hipFree(buf)


def _cm_jobs(L, T, K, rng_seed, parts=False):
    """CpuExperts-style jobs: each token K distinct experts of L in a random order with random weights, plus the shared
    expert on some tokens; with parts, down given as two regions (equal halves, or 1/3 + 2/3 as down_blocks)."""
    r = np.random.default_rng(rng_seed)
    jobs, ojobs = [], []
    bv, bb = moe.BLOCK[L.down_type]
    nb = L.F // bv
    for t in range(T):
        es = r.choice(L.E, size=K, replace=False).tolist() + ([L.E] if t % 3 == 0 else [])
        for e in es:
            g, u, d = L.experts[e] if e < L.E else L.shared
            if e == L.E and (L.sh_gate_type, L.sh_down_type) != (L.gate_type, L.down_type):
                continue
            w = float(r.uniform(0.05, 1.0))
            m = (g, u, d)
            if parts:
                b0 = nb // 2 if e % 2 == 0 or nb < 3 else nb // 3
                rows = d.reshape(L.H, nb * bb)
                d2 = np.ascontiguousarray(np.concatenate([rows[:, :b0 * bb].ravel(), rows[:, b0 * bb:].ravel()]))
                m = (g, u, d2, 2, (0, 0) if b0 == nb // 2 and nb == 2 else (b0, nb - b0))
            jobs.append((m, t, w))
            ojobs.append(((g, u, d), t, w))
    return jobs, ojobs


@pytest.mark.parametrize("T", [1, 8, 64])
@pytest.mark.parametrize("types", [(moe.QT_Q4_K, moe.QT_Q4_K), (moe.QT_IQ3_S, moe.QT_Q8_0), (moe.QT_IQ2_S, moe.QT_Q2_0)])
def test_compute_many_borrowed(T, types):
    """moe_compute_many on borrowed file-layout weights equals the oracle's compute_many bit for bit: T 1 and 8 run
    the decode kernel, 64 the prefill kernels; down given in two parts on some experts (down_parts)."""
    gt, dt = types
    say("compute_many borrowed", moe.TYPE_NAMES[gt], moe.TYPE_NAMES[dt], "T", T)
    L = h.Layer(512, 512, 32, 4, gt, dt, seed=90 + T)
    blk = moe.MoeBlock(512, 512, 32, 4, gt, dt, has_shared=False, max_tokens=64)
    if gt in moe.CODEBOOK_TYPES:
        blk.set_codebooks(h.CODEBOOKS)
    x = h.tokens(91 + T, T, 512)
    for parts in (False, True):
        jobs, ojobs = _cm_jobs(L, T, 4, T + 7, parts)
        y = blk.compute_many(jobs, x)
        yo = h.orc_compute_many(gt, dt, 512, 512, ojobs, x)
        assert np.array_equal(y, yo), (parts, h.max_abs(y, yo))
    blk.close()


@pytest.mark.parametrize("types", [(moe.QT_Q4_K, moe.QT_Q8_0, moe.QT_Q4_K, moe.QT_Q8_0),
                                   (moe.QT_IQ3_S, moe.QT_Q8_0, moe.QT_Q8_0, moe.QT_Q8_0),
                                   (moe.QT_IQ3_S, moe.QT_IQ4_NL, moe.QT_Q8_0, moe.QT_IQ4_NL),
                                   (moe.QT_IQ3_S, moe.QT_Q2_0, moe.QT_Q8_0, moe.QT_Q2_0),
                                   (moe.QT_IQ4_NL, moe.QT_Q2_0, moe.QT_Q2_0, moe.QT_IQ4_NL),
                                   (moe.QT_IQ3_XXS, moe.QT_IQ4_NL, moe.QT_Q4_K, moe.QT_IQ4_NL),
                                   (moe.QT_IQ2_S, moe.QT_Q2_0, moe.QT_Q4_K, moe.QT_IQ4_NL),
                                   (moe.QT_IQ2_S, moe.QT_IQ4_NL, moe.QT_IQ3_XXS, moe.QT_IQ4_NL)])
@pytest.mark.parametrize("T", [1, 8, 100])
def test_model_shape_2560_640(types, T):
    """The reference model's own expert shape (MODEL_LAYER.md:51, :69): n_embd 2560 (ten 256-value units, not a power of
    two), n_ff 640 (down's K two and a half units: its last unit half blocks, half zero padding), with the file's
    types (docs/model/tensors-IQ3_S.tsv: gate/up IQ3_XXS, IQ2_S or IQ3_S, down IQ4_NL or Q2_0, the shared expert's
    gate Q4_K; IQ3_XXS and IQ2_S through the tests' stand-in codebooks) and the 32-value types as gate/up too. Decode
    (T 1, 8) and prefill (T 100) against the oracle, bit for bit."""
    gt, dt, sgt, sdt = types
    say("shape 2560 x 640", [moe.TYPE_NAMES[t] for t in types], "T", T)
    L = h.Layer(2560, 640, 64, 8, gt, dt, sgt, sdt, seed=2560 + T, zipf=1.1)
    blk = L.block(max_tokens=128)
    L.upload(blk)
    x = h.tokens(640 + T, T, 2560)
    y, ids, w = blk.forward(0, x)
    check_block(y, ids, w, *L.oracle_forward(x), blk.bit_exact(T))
    blk.close()


@pytest.mark.parametrize("qtype", [moe.QT_Q8_0, moe.QT_IQ4_NL, moe.QT_Q2_0])
def test_dequantize_partial_unit(tiny_block, qtype):
    """A row of 640 values (two and a half units) through the device layout: the partial unit's blocks decode as the
    format says and nothing past the row is written."""
    m = moe.synth_matrix(5, 2, qtype, 70, 640)
    rb = moe.row_bytes(qtype, 640)
    got = tiny_block.dequantize(qtype, m, 70, 640)
    want = np.stack([h.orc_dequant(qtype, m[r * rb:(r + 1) * rb], 640) for r in range(70)])
    assert np.array_equal(got, want)


def test_codebooks_required_and_checked():
    """IQ3_XXS / IQ2_S contexts refuse to run before moe_set_codebooks; a buffer whose IQ3_S region is not ggml's grid
    (so not the QGRID layout) is refused; after a good buffer the forward runs and matches the oracle."""
    say("codebooks required")
    L = h.Layer(512, 256, 16, 4, moe.QT_IQ3_XXS, moe.QT_IQ4_NL, has_shared=False, seed=77)
    blk = L.block()
    blk.load_router(0, L.router, L.bias)
    for e, (g, u, d) in L.experts.items():
        blk.load_expert(0, e, g, u, d)
    x = h.tokens(78, 2, 512)
    with pytest.raises(moe.MoeError):
        blk.forward(0, x)
    bad = h.CODEBOOKS.copy()
    bad[moe.QGRID_IQ3S] ^= 2
    with pytest.raises(moe.MoeError):
        blk.set_codebooks(bad)
    with pytest.raises(moe.MoeError):
        blk.set_codebooks(h.CODEBOOKS[:moe.QGRID_IQ3S])
    blk.set_codebooks(h.CODEBOOKS)
    y, ids, w = blk.forward(0, x)
    check_block(y, ids, w, *L.oracle_forward(x))
    blk.close()

