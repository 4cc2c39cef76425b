"""Pins the CPU oracle (oracle/oracle.c) before anything is checked against it.

The reference commits no golden vectors for this path (its tests call ggml at run time; docs/TESTING.md:60-74), and
ggml is absent here, so each function is pinned by what the format and the mathematics fix:
  - the IQ3_S grid and kvalues_iq4nl against the sha256s the reference records (docs/spec/QUANT_FORMATS.md:546-547);
  - each decoder on hand-built blocks whose values the format's tables (QUANT_FORMATS.md:176-212, :373-400,
    :447-466, :234-246, :251-262) give position by position;
  - the activation quantisers by their invariants and by exact ties (the rounding rule);
  - the dot products against float64 dots of the decoded operands, to the reference's own tolerance (1e-4 of
    sum |w a|, docs/TESTING.md:45-58), and exactly where every fp32 step is exact;
  - compute against compute_many bit for bit (core/tests/cpu_experts_test.cpp:240-275), y overwritten;
  - the experts and the block against a float64 SwiGLU FFN on the decoded weights;
  - the router against a float64 softmax and a sort with ties to the lower expert (core/tests/topk_test.cpp:60-67).
What only ggml could pin - its SIMD fp32 summation order, its bf16 dot order, the fp32 steps of its CPU Q2_0 dot (a
ggml fork's source the reference does not hold) - is "parity unpinned" (the oracle sums block terms in a stated
canonical order instead, Q2_0 as one term a 32-value half like the CUDA kernel).
"""
import hashlib

import numpy as np
import pytest

from tests import harness as h
from tests.harness import moe

rng = np.random.default_rng(20261201)


def f16(v):
    return np.frombuffer(np.float16(v).tobytes(), dtype=np.uint8)


# --------------------------------------------------------------------------------------------------------------
# Scalars and the codebook


def test_iq3s_grid_matches_pinned_sha256():
    g = h.orc_grid()
    assert hashlib.sha256(g.astype("<u4").tobytes()).hexdigest() == (
        "bd1af4945a1717c65610b0284e4628b9a1ba3b306fae3a06f6e5f597356e349f")
    b = g.view(np.uint8)
    assert set(np.unique(b).tolist()) == {1, 3, 5, 7, 9, 11, 13, 15}
    assert len(np.unique(g)) == 512


def test_iq4nl_values_match_pinned_sha256():
    v = h.orc_iq4nl()
    assert hashlib.sha256(v.tobytes()).hexdigest() == (
        "61aa47540aa024b5d6ddaa839b84ffe59f3d5a349af5c6c7ffcb5e0474b46163")
    assert v[0] == -127 and v[-1] == 113 and (np.diff(v.astype(int)) > 0).all()


def test_fp16_conversions_match_ieee():
    allh = np.arange(65536, dtype=np.uint16)
    want = allh.view(np.float16).astype(np.float32)
    got = np.array([h.oracle.orc_fp16_to_fp32(int(v)) for v in allh[::7]], dtype=np.float32)
    w = want[::7]
    ok = (got.view(np.uint32) == w.view(np.uint32)) | (np.isnan(got) & np.isnan(w))
    assert ok.all()
    xs = np.concatenate([rng.standard_normal(20000).astype(np.float32) * s for s in (1e-7, 1e-5, 1e-3, 1, 1e3, 7e4)])
    # exact ties between two halves: 1 + 2^-11 (round to even: 1.0), 1 + 3 2^-11 (to 1 + 2^-9)
    xs = np.concatenate([xs, np.array([1 + 2**-11, 1 + 3 * 2**-11, 65504, 65519.99, 65520, 2**-25, 3 * 2**-26],
                                      dtype=np.float32)])
    got = np.array([h.oracle.orc_fp32_to_fp16(float(v)) for v in xs], dtype=np.uint16)
    assert np.array_equal(got, xs.astype(np.float16).view(np.uint16))


def test_bf16_is_nearest_even():
    xs = rng.standard_normal(5000).astype(np.float32) * np.float32(3.0)
    xs[:4] = np.array([1 + 2**-8, 1 + 3 * 2**-8, -(1 + 2**-8), 1.5], dtype=np.float32)  # ties
    assert h.oracle.orc_fp32_to_bf16(0.0) == 0
    for v in xs[xs != 0]:
        b = h.oracle.orc_fp32_to_bf16(float(v))
        got = float(h.bf16_to_f32(np.array([b], dtype=np.uint16))[0])
        lo = float(h.bf16_to_f32(np.array([b - 1], dtype=np.uint16))[0])
        hi = float(h.bf16_to_f32(np.array([b + 1], dtype=np.uint16))[0])
        d = abs(float(v) - got)
        assert d <= abs(float(v) - lo) and d <= abs(float(v) - hi)
        if d == abs(float(v) - lo) or d == abs(float(v) - hi):
            assert b % 2 == 0  # a tie went to the even one
    assert h.oracle.orc_fp32_to_bf16(1 + 2**-8) == 0x3F80
    assert h.oracle.orc_fp32_to_bf16(1 + 3 * 2**-8) == 0x3F82


# --------------------------------------------------------------------------------------------------------------
# Decoders, position by position


def test_q8_0_decoder():
    q = np.arange(-16, 16, dtype=np.int8)
    blk = np.concatenate([f16(0.5), q.view(np.uint8)])
    y = h.orc_dequant(moe.QT_Q8_0, blk, 32)
    assert np.array_equal(y, (np.float32(0.5) * q.astype(np.float32)))


def test_iq4_nl_decoder():
    """Byte j holds value j in its low nibble and value j + 16 in its high one; y = d kvalues[nibble]."""
    kv = h.orc_iq4nl().astype(np.float32)
    lo = np.arange(16, dtype=np.uint8)
    hi = (np.arange(16, dtype=np.uint8) * 7 + 3) % 16
    blk = np.concatenate([f16(0.25), lo | (hi << 4)]).astype(np.uint8)
    y = h.orc_dequant(moe.QT_IQ4_NL, blk, 32)
    assert np.array_equal(y, np.float32(0.25) * np.concatenate([kv[lo], kv[hi]]))


def test_q2_0_decoder():
    """Value j is bits 2 (j mod 4), 2 (j mod 4) + 1 of byte j / 4; y = (q - 1) d: codes mean -1, 0, 1, 2."""
    q = rng.integers(0, 4, size=64)
    qs = np.zeros(16, dtype=np.uint8)
    for j in range(64):
        qs[j // 4] |= np.uint8(q[j] << (2 * (j % 4)))
    y = h.orc_dequant(moe.QT_Q2_0, np.concatenate([f16(-1.5), qs]), 64)
    assert np.array_equal(y, (q - 1).astype(np.float32) * np.float32(-1.5))
    assert np.array_equal(h.orc_dequant(moe.QT_Q2_0, np.concatenate([f16(2.0), np.full(16, 0xE4, np.uint8)]), 64),
                          np.tile(np.array([-2, 0, 2, 4], np.float32), 16))  # 0xE4: codes 0, 1, 2, 3


def test_iq3_xxs_decoder():
    """Sub-block b: index bytes 8 b .. 8 b + 7 (groups of four values), then its word: four 7-bit sign indices (the
    eighth sign the parity) and the scale s in bits 28-31; y = ((d (0.5 + s)) 0.5) grid sign. The grid is the tests'
    stand-in table (h.CODEBOOKS)."""
    grid = h.CODEBOOKS[moe.QGRID_IQ3XXS:moe.QGRID_IQ3XXS + 1024].view("<u4")
    idx = rng.integers(0, 256, size=64)
    s = rng.integers(0, 16, size=8)
    s7 = rng.integers(0, 128, size=(8, 4))
    words = np.zeros(8, np.uint32)
    for b in range(8):
        words[b] = (int(s[b]) << 28) | sum(int(s7[b, l]) << (7 * l) for l in range(4))
    blk = np.concatenate([f16(0.125), idx.astype(np.uint8), words.view(np.uint8)])
    y = h.orc_dequant(moe.QT_IQ3_XXS, blk, 256)
    d = np.float32(0.125)
    for v in range(256):
        b, j = v // 32, v % 32
        l = j // 8
        sb = int(s7[b, l]) | ((bin(int(s7[b, l])).count("1") & 1) << 7)
        mag = (int(grid[idx[8 * b + 2 * l + (j % 8) // 4]]) >> (8 * (j % 4))) & 0xFF
        db = np.float32(np.float32(d * np.float32(0.5 + s[b])) * np.float32(0.5))
        want = np.float32(db * np.float32(mag)) * (-1 if (sb >> (j % 8)) & 1 else 1)
        assert y[v] == want, v


def test_iq2_s_decoder():
    """Group g of sub-block b: index qs[4 b + g] | ((qh[b] >> 2 g) & 3) << 8, sign byte signs[4 b + g], scale the low
    nibble of scales[b] for values 0-15 and the high for 16-31; y = ((d (0.5 + s)) 0.25) grid sign."""
    grid = h.CODEBOOKS[moe.QGRID_IQ2S:moe.QGRID_IQ2S + 8192].view("<u8")
    qs = rng.integers(0, 256, size=32).astype(np.uint8)
    sg = rng.integers(0, 256, size=32).astype(np.uint8)
    qh = rng.integers(0, 256, size=8).astype(np.uint8)
    sc = rng.integers(0, 256, size=8).astype(np.uint8)
    blk = np.concatenate([f16(0.25), qs, sg, qh, sc])
    y = h.orc_dequant(moe.QT_IQ2_S, blk, 256)
    for v in range(256):
        b, j = v // 32, v % 32
        g = j // 8
        ix = int(qs[4 * b + g]) | (((int(qh[b]) >> (2 * g)) & 3) << 8)
        mag = (int(grid[ix]) >> (8 * (j % 8))) & 0xFF
        s = (int(sc[b]) >> (4 * (j // 16))) & 15
        db = np.float32(np.float32(np.float32(0.25) * np.float32(0.5 + s)) * np.float32(0.25))
        want = np.float32(db * np.float32(mag)) * (-1 if (int(sg[4 * b + g]) >> (j % 8)) & 1 else 1)
        assert y[v] == want, v


def pack_q4_k_scales(sc, m):
    """QUANT_FORMATS.md's table for the 12 scale bytes (bytes 0-3, 4-7, 8-11)."""
    b = np.zeros(12, dtype=np.uint8)
    for j in range(4):
        b[j] = (sc[j] & 63) | ((sc[j + 4] >> 4) << 6)
        b[j + 4] = (m[j] & 63) | ((m[j + 4] >> 4) << 6)
        b[j + 8] = (sc[j + 4] & 15) | ((m[j + 4] & 15) << 4)
    return b


def test_q4_k_decoder():
    sc = [3, 17, 33, 63, 20, 36, 50, 61]
    m = [5, 18, 40, 63, 22, 33, 47, 60]
    q = (np.arange(256) * 7 + 3) % 16
    qs = np.zeros(128, dtype=np.uint8)
    for c in range(4):  # chunk c, byte l: low nibble value 64c + l, high nibble value 64c + 32 + l
        for l in range(32):
            qs[32 * c + l] = q[64 * c + l] | (q[64 * c + 32 + l] << 4)
    d, dmin = np.float32(0.25), np.float32(0.125)
    blk = np.concatenate([f16(d), f16(dmin), pack_q4_k_scales(sc, m), qs])
    y = h.orc_dequant(moe.QT_Q4_K, blk, 256)
    want = np.empty(256, dtype=np.float32)
    for v in range(256):
        j = v // 32
        want[v] = (d * np.float32(sc[j])) * np.float32(q[v]) - dmin * np.float32(m[j])
    assert np.array_equal(y, want)


def build_iq3s(idx, signs_bits, s, d):
    """An IQ3_S block from 64 grid indices (9 bits), 256 sign bits and 8 scales, by the format's table."""
    qs = np.array([i & 255 for i in idx], dtype=np.uint8)
    qh = np.zeros(8, dtype=np.uint8)
    for k, i in enumerate(idx):
        qh[k // 8] |= ((i >> 8) & 1) << (k % 8)
    sg = np.zeros(32, dtype=np.uint8)
    for b in range(8):
        for v in range(32):  # bit j of byte 4b + l is the sign of value 8l + j of sub-block b
            if signs_bits[32 * b + v]:
                sg[4 * b + v // 8] |= 1 << (v % 8)
    scales = np.array([s[2 * c] | (s[2 * c + 1] << 4) for c in range(4)], dtype=np.uint8)
    return np.concatenate([f16(d), qs, qh, sg, scales])


def test_iq3_s_decoder():
    grid = h.orc_grid().view(np.uint8).reshape(512, 4)
    idx = [(37 * k + 11) % 512 for k in range(64)]
    assert any(i >= 256 for i in idx) and any(i < 256 for i in idx)
    signs = rng.integers(0, 2, 256)
    s = [0, 1, 5, 15, 7, 3, 9, 12]
    d = np.float32(0.0078125)
    y = h.orc_dequant(moe.QT_IQ3_S, build_iq3s(idx, signs, s, d), 256)
    want = np.empty(256, dtype=np.float32)
    for v in range(256):
        b, k, j = v // 32, v // 4, v % 4
        db = d * np.float32(1 + 2 * s[b])
        want[v] = db * np.float32(grid[idx[k], j]) * np.float32(-1 if signs[v] else 1)
    assert np.array_equal(y, want)


def test_q5_k_decoder():
    """Q4_K's scales and nibbles (chunk c, byte l: values 64c + l and 64c + 32 + l) plus qh: bit k of byte l is bit 4 of
    value 32 k + l (QUANT_FORMATS.md:401-417); y = (d sc) q - dmin m with q = nibble + 16 bit."""
    sc = [1, 17, 33, 63, 20, 36, 50, 61]
    m = [5, 18, 40, 63, 0, 33, 47, 60]
    q = (np.arange(256) * 11 + 5) % 32
    qs = np.zeros(128, dtype=np.uint8)
    for c in range(4):
        for l in range(32):
            qs[32 * c + l] = (q[64 * c + l] & 15) | ((q[64 * c + 32 + l] & 15) << 4)
    qh = np.zeros(32, dtype=np.uint8)
    for v in range(256):
        qh[v % 32] |= ((q[v] >> 4) & 1) << (v // 32)
    d, dmin = np.float32(0.5), np.float32(0.0625)
    blk = np.concatenate([f16(d), f16(dmin), pack_q4_k_scales(sc, m), qh, qs])
    assert blk.size == 176
    y = h.orc_dequant(moe.QT_Q5_K, blk, 256)
    want = np.array([(d * np.float32(sc[v // 32])) * np.float32(q[v]) - dmin * np.float32(m[v // 32])
                     for v in range(256)], dtype=np.float32)
    assert np.array_equal(y, want)


def test_q6_k_decoder():
    """QUANT_FORMATS.md:419-445 position by position: value v (h = v / 128, l = v % 32) takes its low four bits from
    ql[64h + l] (low nibble: v - 128h < 32; high nibble: 64..95), ql[64h + 32 + l] (32..63 low, 96..127 high), its high
    two bits from qh[32h + l] at bits 0, 2, 4, 6 for the four 32-value quarters; scales[v / 16] signed; d last;
    y = (d sc) (q - 32)."""
    q = (np.arange(256) * 37 + 9) % 64
    ql = np.zeros(128, dtype=np.uint8)
    qh = np.zeros(64, dtype=np.uint8)
    for v in range(256):
        hh, r, l = v // 128, v % 128, v % 32
        quarter = r // 32
        byte = 64 * hh + (32 if quarter in (1, 3) else 0) + l
        ql[byte] |= (q[v] & 15) << (4 if quarter >= 2 else 0)
        qh[32 * hh + l] |= (q[v] >> 4) << (2 * quarter)
    scales = np.array([-128, -77, -1, 0, 1, 5, 33, 127, -20, 64, -64, 100, -100, 2, -2, 90], dtype=np.int8)
    d = np.float32(2.0 ** -7 * 1.5)
    blk = np.concatenate([ql, qh, scales.view(np.uint8), f16(d)])
    assert blk.size == 210
    y = h.orc_dequant(moe.QT_Q6_K, blk, 256)
    want = np.array([(d * np.float32(scales[v // 16])) * np.float32(q[v] - 32) for v in range(256)], dtype=np.float32)
    assert np.array_equal(y, want)


def test_iq4_xs_decoder():
    """d, then scales_h (bits 2b, 2b + 1: bits 4-5 of sub-block b's scale), scales_l (byte b / 2, low nibble for even
    b), then 16 qs bytes a sub-block (byte j: value j low, j + 16 high) (QUANT_FORMATS.md:213-232);
    y = (d (ls - 32)) kvalues[nibble]."""
    kv = h.orc_iq4nl().astype(np.float32)
    ls = [0, 63, 32, 31, 1, 47, 16, 40]
    sh = sum(((l >> 4) & 3) << (2 * b) for b, l in enumerate(ls))
    sl = np.array([(ls[2 * i] & 15) | ((ls[2 * i + 1] & 15) << 4) for i in range(4)], dtype=np.uint8)
    nib = (np.arange(256) * 5 + 3) % 16
    qs = np.zeros(128, dtype=np.uint8)
    for b in range(8):
        for j in range(16):
            qs[16 * b + j] = nib[32 * b + j] | (nib[32 * b + j + 16] << 4)
    d = np.float32(-0.03125)
    blk = np.concatenate([f16(d), np.frombuffer(np.uint16(sh).tobytes(), np.uint8), sl, qs])
    assert blk.size == 136
    y = h.orc_dequant(moe.QT_IQ4_XS, blk, 256)
    want = np.array([(d * np.float32(ls[v // 32] - 32)) * kv[nib[v]] for v in range(256)], dtype=np.float32)
    assert np.array_equal(y, want)


# --------------------------------------------------------------------------------------------------------------
# Activation quantisers


def q8k_fields(buf, nb):
    b = buf.reshape(nb, 292)
    d = b[:, :4].copy().view(np.float32).ravel()
    qs = b[:, 4:260].copy().view(np.int8)
    bs = b[:, 260:292].copy().view(np.int16)
    return d, qs, bs


def test_q8_k_invariants_and_ties():
    x = rng.standard_normal(1024).astype(np.float32)
    d, qs, bs = q8k_fields(h.orc_quant_act(moe.QT_Q8_K, x), 4)
    xb = x.reshape(4, 256)
    for i in range(4):
        j = np.argmax(np.abs(xb[i]))
        assert qs[i, j] == -127  # iscale = -127 / max: the largest magnitude takes -127
        assert np.all(np.abs(qs[i].astype(np.float32) * d[i] - xb[i]) <= np.abs(d[i]) * 0.5000001 + 1e-7)
        assert np.array_equal(bs[i], qs[i].reshape(16, 16).astype(np.int32).sum(1).astype(np.int16))
        assert np.sign(d[i]) == -np.sign(xb[i, j])
    # max = -127 gives iscale = 1: exact ties round to even
    t = np.zeros(256, dtype=np.float32)
    t[:5] = [-127.0, 2.5, 3.5, -2.5, 0.5]
    d, qs, _ = q8k_fields(h.orc_quant_act(moe.QT_Q8_K, t), 1)
    assert d[0] == 1.0 and list(qs[0, :5]) == [-127, 2, 4, -2, 0]
    d, qs, bs = q8k_fields(h.orc_quant_act(moe.QT_Q8_K, np.zeros(256, np.float32)), 1)
    assert d[0] == 0 and not qs.any() and not bs.any()


def test_q8_0_invariants_and_ties():
    x = rng.standard_normal(256).astype(np.float32)
    b = h.orc_quant_act(moe.QT_Q8_0, x).reshape(8, 34)
    for i in range(8):
        xb = x[32 * i:32 * i + 32]
        amax = np.float32(np.abs(xb).max())
        assert b[i, :2].copy().view(np.float16)[0] == np.float16(amax / np.float32(127))
        q = b[i, 2:].copy().view(np.int8)
        assert q[np.argmax(np.abs(xb))] in (127, -127)
        dd = float(amax / np.float32(127))
        assert np.all(np.abs(q * dd - xb) <= dd * 0.5000001)
    t = np.zeros(32, dtype=np.float32)
    t[:4] = [127.0, 2.5, 3.5, -2.5]  # amax 127: scale 1, ties to even
    q = h.orc_quant_act(moe.QT_Q8_0, t)[2:].view(np.int8)
    assert list(q[:4]) == [127, 2, 4, -2]


# --------------------------------------------------------------------------------------------------------------
# Dot products


def random_blocks(qtype, n):
    """n blocks of random bytes with scales set so values stay small (core/tests/test_util.h:62-103's rule)."""
    nv, nbytes = moe.BLOCK[qtype]
    b = rng.integers(0, 256, size=(n, nbytes), dtype=np.uint8)
    reach = {moe.QT_Q8_0: [(0, 128)], moe.QT_Q4_K: [(0, 63 * 15), (2, 63)], moe.QT_IQ3_S: [(0, 31 * 15)],
             moe.QT_IQ4_NL: [(0, 127)], moe.QT_Q2_0: [(0, 2)], moe.QT_IQ3_XXS: [(0, 62 * 31)],
             moe.QT_IQ2_S: [(0, 43 * 31)], moe.QT_Q5_K: [(0, 63 * 31), (2, 63)], moe.QT_Q6_K: [(208, 127 * 32)],
             moe.QT_IQ4_XS: [(0, 31 * 127)]}[qtype]
    for k in range(n):
        for off, r in reach:
            v = np.ldexp(1.0 + rng.integers(0, 1024) / 1024.0, int(rng.integers(0, 3)) - 5) / r
            b[k, off:off + 2] = f16(v * (1 if qtype != moe.QT_Q4_K or off == 0 else 1))
    return b.ravel()


@pytest.mark.parametrize("qtype", [moe.QT_Q8_0, moe.QT_Q4_K, moe.QT_IQ3_S, moe.QT_IQ4_NL, moe.QT_Q2_0, moe.QT_IQ3_XXS,
                                   moe.QT_IQ2_S, moe.QT_Q5_K, moe.QT_Q6_K, moe.QT_IQ4_XS])
@pytest.mark.parametrize("n", [256, 2048])
def test_vec_dot_against_decoded_float64(qtype, n):
    for trial in range(20):
        w = random_blocks(qtype, n // moe.BLOCK[qtype][0]) if trial % 2 else moe.synth_matrix(trial, 5, qtype, 1, n)
        x = rng.standard_normal(n).astype(np.float32)
        at = h.vec_dot_type(qtype)
        a = h.orc_quant_act(at, x)
        wd = h.orc_dequant(qtype, w, n).astype(np.float64)
        ad = act_decode(at, a, n)
        ref = float(np.dot(wd, ad))
        got = h.orc_vec_dot(qtype, n, w, a)
        assert abs(got - ref) <= 1e-4 * float(np.abs(wd * ad).sum()) + 1e-30


def act_decode(at, a, n):
    if at == moe.QT_Q8_0:
        b = a.reshape(n // 32, 34)
        d = b[:, :2].copy().view(np.float16).astype(np.float64)
        return (b[:, 2:].copy().view(np.int8).astype(np.float64) * d).ravel()
    d, qs, _ = q8k_fields(a, n // 256)
    return (qs.astype(np.float64) * d[:, None].astype(np.float64)).ravel()


def test_vec_dot_exact_when_every_step_is_exact():
    """Power-of-two scales and small codes: every fp32 product and sum is exact, so the dot must equal the exact
    integer dot times the scales, whatever the order. Pins the integer part (indices, signs, scales, minimums)."""
    n = 1024
    # Q8_0 against q8_0
    w = np.zeros((n // 32, 34), dtype=np.uint8)
    w[:, :2] = f16(2.0**-6)
    w[:, 2:] = rng.integers(-20, 21, size=(n // 32, 32), dtype=np.int8).view(np.uint8)
    a = np.zeros((n // 32, 34), dtype=np.uint8)
    a[:, :2] = f16(2.0**-3)
    a[:, 2:] = rng.integers(-20, 21, size=(n // 32, 32), dtype=np.int8).view(np.uint8)
    exact = float((w[:, 2:].view(np.int8).astype(np.int64) * a[:, 2:].view(np.int8).astype(np.int64)).sum()) * 2.0**-9
    assert h.orc_vec_dot(moe.QT_Q8_0, n, w.ravel(), a.ravel()) == exact
    # IQ4_NL and Q2_0 against the same q8_0 blocks: codebook values and codes q - 1, scale 2^-6
    ad = a[:, 2:].view(np.int8).astype(np.int64).ravel()
    kv = h.orc_iq4nl().astype(np.int64)
    nib = rng.integers(0, 16, size=(n // 32, 32))
    w4 = np.zeros((n // 32, 18), dtype=np.uint8)
    w4[:, :2] = f16(2.0**-6)
    w4[:, 2:] = (nib[:, :16] | (nib[:, 16:] << 4)).astype(np.uint8)
    assert h.orc_vec_dot(moe.QT_IQ4_NL, n, w4.ravel(), a.ravel()) == float((kv[nib].ravel() * ad).sum()) * 2.0**-9
    q2 = rng.integers(0, 4, size=(n // 64, 64))
    w2 = np.zeros((n // 64, 18), dtype=np.uint8)
    w2[:, :2] = f16(2.0**-6)
    for j in range(64):
        w2[:, 2 + j // 4] |= (q2[:, j] << (2 * (j % 4))).astype(np.uint8)
    assert h.orc_vec_dot(moe.QT_Q2_0, n, w2.ravel(), a.ravel()) == float(((q2 - 1).ravel() * ad).sum()) * 2.0**-9
    # Q4_K and IQ3_S against q8_K with d = 2^-4
    x = rng.integers(-20, 21, size=n).astype(np.float32)
    x[::256] = -127.0  # max = -127: iscale = 1, codes = x, d = 1
    aq = h.orc_quant_act(moe.QT_Q8_K, x)
    for qtype in (moe.QT_Q4_K, moe.QT_IQ3_S, moe.QT_IQ3_XXS, moe.QT_IQ2_S, moe.QT_Q5_K, moe.QT_Q6_K, moe.QT_IQ4_XS):
        wq = random_blocks(qtype, n // 256).reshape(n // 256, -1)
        wq[:, 208 if qtype == moe.QT_Q6_K else 0:][:, :2] = f16(2.0**-4)
        if qtype in (moe.QT_Q4_K, moe.QT_Q5_K):
            wq[:, 2:4] = f16(2.0**-5)
        wd = h.orc_dequant(qtype, wq.ravel(), n).astype(np.float64)
        assert h.orc_vec_dot(qtype, n, wq.ravel(), aq) == float(np.dot(wd, x.astype(np.float64)))


# --------------------------------------------------------------------------------------------------------------
# The experts


def dense_ffn(gate, up, down, gt, dt, H, F, x, limit=0.0):
    G = h.orc_dequant(gt, gate, F * H).reshape(F, H).astype(np.float64)
    U = h.orc_dequant(gt, up, F * H).reshape(F, H).astype(np.float64)
    D = h.orc_dequant(dt, down, H * F).reshape(H, F).astype(np.float64)
    g, u = G @ x.astype(np.float64), U @ x.astype(np.float64)
    if limit > 0:
        g, u = np.minimum(g, limit), np.clip(u, -limit, limit)
    return D @ (g / (1 + np.exp(-g)) * u)


TYPES = [(moe.QT_Q8_0, moe.QT_Q8_0), (moe.QT_Q4_K, moe.QT_Q4_K), (moe.QT_IQ3_S, moe.QT_Q4_K), (moe.QT_IQ3_S, moe.QT_IQ3_S),
         (moe.QT_Q4_K, moe.QT_Q8_0), (moe.QT_Q4_K, moe.QT_IQ4_NL), (moe.QT_IQ4_NL, moe.QT_Q2_0),
         (moe.QT_IQ3_XXS, moe.QT_IQ4_NL), (moe.QT_IQ2_S, moe.QT_Q2_0), (moe.QT_Q5_K, moe.QT_Q6_K),
         (moe.QT_IQ4_XS, moe.QT_Q5_K), (moe.QT_Q6_K, moe.QT_IQ4_XS)]


@pytest.mark.parametrize("gt,dt", TYPES)
def test_compute_many_against_dense_and_compute(gt, dt):
    H, F, T = 512, 256, 3
    ex = [(moe.synth_matrix(1, 10 * e, gt, F, H), moe.synth_matrix(1, 10 * e + 1, gt, F, H),
           moe.synth_matrix(1, 10 * e + 2, dt, H, F)) for e in range(3)]
    x = h.tokens(3, T, H)
    jobs = [(ex[0], 0, 0.5), (ex[1], 0, 0.25), (ex[1], 1, 0.75), (ex[2], 1, 0.125), (ex[1], 2, 1.0)]
    y = h.orc_compute_many(gt, dt, H, F, jobs, x)
    assert np.isfinite(y).all()  # y overwritten (it started as NaN)
    for t in range(T):
        ref = sum(w * dense_ffn(*m, gt, dt, H, F, x[t]) for m, tt, w in jobs if tt == t)
        assert h.rel_l2(y[t], ref) < 3e-2, (t, h.rel_l2(y[t], ref))
    # compute (one token, experts in order) = compute_many's row for that token, bit for bit
    import ctypes as C
    for t in range(T):
        mine = [(m, w) for m, tt, w in jobs if tt == t]
        n = len(mine)
        gp = (C.c_void_p * n)(*[m[0].ctypes.data for m, _ in mine])
        upp = (C.c_void_p * n)(*[m[1].ctypes.data for m, _ in mine])
        dp = (C.c_void_p * n)(*[m[2].ctypes.data for m, _ in mine])
        w = np.array([w for _, w in mine], dtype=np.float32)
        s = h.OrcShape(gt, dt, H, F, 0.0)
        y1 = np.empty(H, dtype=np.float32)
        assert h.oracle.orc_compute(C.byref(s), gp, upp, dp, h.ptr(w), n, h.ptr(np.ascontiguousarray(x[t])),
                                    h.ptr(y1)) == 0
        assert np.array_equal(y1, y[t])
    # threads change nothing
    assert np.array_equal(y, h.orc_compute_many(gt, dt, H, F, jobs, x, nthreads=1))


@pytest.mark.parametrize("gt,ut", [(moe.QT_Q4_K, moe.QT_IQ4_XS), (moe.QT_Q6_K, moe.QT_Q5_K), (moe.QT_IQ4_XS, moe.QT_Q6_K)])
def test_compute_many_with_up_of_another_type(gt, ut):
    """A shared expert whose up differs from its gate in type (the model file's blk.0: Q4_K gate, IQ4_XS up): the
    dense FFN on the decoded weights, and the same bits as a gate/up pair of one type where the two agree."""
    import ctypes as C
    H, F, T, dt = 512, 256, 2, moe.QT_IQ4_NL
    g = moe.synth_matrix(5, 1, gt, F, H)
    u = moe.synth_matrix(5, 2, ut, F, H)
    d = moe.synth_matrix(5, 3, dt, H, F)
    x = h.tokens(6, T, H)
    jobs = (h.OrcJob * T)(*[h.OrcJob(h.ptr(g), h.ptr(u), h.ptr(d), t, 1.0) for t in range(T)])
    y = np.empty((T, H), dtype=np.float32)
    s = h.OrcShape(gt, dt, H, F, 0.0, ut)
    assert h.oracle.orc_compute_many(C.byref(s), jobs, T, T, h.ptr(x), H, h.ptr(y), H, 1) == 0
    G = h.orc_dequant(gt, g, F * H).reshape(F, H).astype(np.float64)
    U = h.orc_dequant(ut, u, F * H).reshape(F, H).astype(np.float64)
    D = h.orc_dequant(dt, d, H * F).reshape(H, F).astype(np.float64)
    for t in range(T):
        a, b = G @ x[t], U @ x[t]
        ref = D @ (a / (1 + np.exp(-a)) * b)
        assert h.rel_l2(y[t], ref) < 3e-2
    s_bad = h.OrcShape(gt, dt, H, F, 0.0, moe.QT_Q8_0)  # q8_0 up against a q8_K gate: refused
    assert h.oracle.orc_compute_many(C.byref(s_bad), jobs, T, T, h.ptr(x), H, h.ptr(y), H, 1) == -1


def test_compute_many_no_jobs_and_swiglu_limit():
    H, F = 512, 256
    x = h.tokens(4, 2, H)
    y = h.orc_compute_many(moe.QT_Q8_0, moe.QT_Q8_0, H, F, [], x)
    assert not y.any()
    m = tuple(moe.synth_matrix(2, s, moe.QT_Q8_0, r, c, 0.05) for s, r, c in ((0, F, H), (1, F, H), (2, H, F)))
    L = 0.3
    y = h.orc_compute_many(moe.QT_Q8_0, moe.QT_Q8_0, H, F, [(m, 0, 1.0)], x[:1], swiglu_limit=L)
    ref = dense_ffn(*m, moe.QT_Q8_0, moe.QT_Q8_0, H, F, x[0], limit=L)
    assert h.rel_l2(y[0], ref) < 3e-2
    y0 = h.orc_compute_many(moe.QT_Q8_0, moe.QT_Q8_0, H, F, [(m, 0, 1.0)], x[:1])
    assert h.rel_l2(y0[0], ref) > 0.05  # the clamp is live at this L


# --------------------------------------------------------------------------------------------------------------
# The router and the block


def test_router_against_float64_and_sort():
    H, E, K, T = 512, 64, 6, 5
    L = h.Layer(H, 256, E, K, moe.QT_Q8_0, moe.QT_Q8_0, seed=9, experts=[], zipf=1.1)
    x = h.tokens(9, T, H)
    lg, ids, w = L.oracle_route(x)
    xb = h.bf16_to_f32(h.to_bf16(x)).astype(np.float64)
    W = h.bf16_to_f32(L.router).astype(np.float64)
    ref = (W @ xb.T).T.astype(np.float32)
    ref[:, :E] = ref[:, :E] + L.bias
    assert np.array_equal(lg, ref)
    for t in range(T):
        order = np.lexsort((np.arange(E), -lg[t, :E].astype(np.float64)))[:K]
        assert np.array_equal(ids[t], order)
        p = np.exp(lg[t, :E].astype(np.float64) - lg[t, :E].max())
        p /= p.sum()
        ww = p[order] / p[order].sum()
        assert np.allclose(w[t], ww, rtol=2e-6, atol=0)


def test_router_ties_go_to_the_lower_expert():
    H, E, K = 512, 16, 4
    L = h.Layer(H, 256, E, K, moe.QT_Q8_0, moe.QT_Q8_0, seed=3, experts=[])
    L.router[[2, 5, 11]] = L.router[7]  # four experts with one logit
    L.router[[3, 9]] = L.router[0]
    x = h.tokens(3, 8, H)
    lg, ids, _ = L.oracle_route(x)
    for t in range(8):
        order = sorted(range(E), key=lambda e: (-float(lg[t, e]), e))[:K]
        assert list(ids[t]) == order


def test_block_reduces_to_dense_ffn_when_k_is_all_and_experts_equal():
    """k = E with every expert the same: y = (sum_k w_k) FFN(x) + gs s = FFN(x) (1 + gs) up to rounding."""
    H, F, E = 512, 256, 4
    L = h.Layer(H, F, E, E, moe.QT_Q4_K, moe.QT_Q4_K, seed=5, experts=[0])
    for e in range(1, E):
        L.experts[e] = L.experts[0]
    L.shared = L.experts[0]
    x = h.tokens(5, 2, H)
    y, ids, w = L.oracle_forward(x)
    lg, _, _ = L.oracle_route(x)
    for t in range(2):
        gs = 1 / (1 + np.exp(-float(lg[t, E])))
        ref = dense_ffn(*L.experts[0], moe.QT_Q4_K, moe.QT_Q4_K, H, F, x[t]) * (float(w[t].sum()) + gs)
        assert h.rel_l2(y[t], ref) < 3e-2
        assert sorted(ids[t].tolist()) == list(range(E))


# --------------------------------------------------------------------------------------------------------------
# The hyper-connection mix and combine


def test_hc_mix_against_float64_and_closed_forms():
    """orc_hc_pre against a float64 restatement of MODEL_LAYER.md 1.1 (bf16 roundings included) to 1e-5, and two
    closed forms: with W_up = 0 every gate is sigma(0) = 1/2, so x = (sum_s n_s / 2) / 4 exactly as the fp32 steps
    give it; with W_inject = 0 the combine is R_s + y bit for bit (2 sigma(0) = 1)."""
    H, lr, T = 512, 64, 3
    hc = h.HcModule(H, lr, seed=3)
    R = rng.standard_normal((T, 4, H)).astype(np.float32)
    x, inj = hc.pre(R)
    bf = lambda a: h.bf16_to_f32(h.to_bf16(np.asarray(a, np.float32))).astype(np.float64)
    Wd, Wi, Wu = (h.bf16_to_f32(m).astype(np.float64) for m in (hc.down, hc.inj, hc.up))
    for t in range(T):
        r = R[t].astype(np.float64)
        n = r / np.sqrt((r * r).mean(axis=1, keepdims=True) + 1e-6) * hc.gamma.reshape(4, H)
        z = Wd @ bf(n.ravel()) / 4
        l = z / (1 + np.exp(-z))
        a = (Wu @ bf(l)).reshape(4, H)
        want = (n / (1 + np.exp(-a))).sum(axis=0) / 4
        assert np.allclose(x[t], want, rtol=1e-5, atol=1e-6)
        assert np.allclose(inj[t], Wi @ bf(n.ravel()), rtol=1e-5, atol=1e-6)
    hc0 = h.HcModule(H, lr, seed=3)
    hc0.up[:] = 0
    x0, _ = hc0.pre(R)
    for t in range(T):
        r = R[t]
        acc = np.zeros(H, np.float32)
        for s in range(4):
            ss = float(np.sum((r[s] * r[s]).astype(np.float64)))  # fp32 squares summed in double (exact here)
            scale = np.float32(1.0) / np.sqrt(np.float32(np.float32(ss / H) + np.float32(1e-6)), dtype=np.float32)
            n = (r[s] * scale) * hc0.gamma[s * H:(s + 1) * H]
            acc = acc + n * np.float32(0.5)
        assert np.array_equal(x0[t], acc * np.float32(0.25))
    y = rng.standard_normal((T, H)).astype(np.float32)
    assert np.array_equal(h.HcModule.post(R, np.zeros((T, 4), np.float32), y), R + y[:, None, :])


def test_forward_resident_reduces_to_its_parts():
    """The hybrid oracle (experts off the device summed apart, after gs s): with every expert resident it is the plain
    block bit for bit; with none resident and no shared expert it is compute_many over the token's jobs in rank order
    (CpuExperts::compute_many's sum, core/cpu/experts.h:32-60)."""
    import ctypes as C

    def resident_forward(L, resident, x):
        Lo, keep = L._orc_layer()
        y = np.empty((x.shape[0], L.H), dtype=np.float32)
        r = np.ascontiguousarray(resident, dtype=np.uint8)
        assert h.oracle.orc_moe_forward_resident(C.byref(Lo), h.ptr(r), h.ptr(x), x.shape[0], L.H, h.ptr(y), L.H,
                                                 4) == 0
        del keep
        return y

    L = h.Layer(512, 256, 16, 4, moe.QT_Q4_K, moe.QT_Q8_0, seed=17, zipf=1.1)
    x = h.tokens(5, 6, 512)
    assert np.array_equal(resident_forward(L, np.ones(16, np.uint8), x), L.oracle_forward(x)[0])
    L0 = h.Layer(512, 256, 16, 4, moe.QT_Q4_K, moe.QT_Q8_0, seed=18, zipf=1.1, has_shared=False)
    y = resident_forward(L0, np.zeros(16, np.uint8), x)
    _, ids, w = L0.oracle_route(x)
    jobs = [(L0.experts[int(ids[t, k])], t, float(w[t, k])) for t in range(6) for k in range(4)]
    assert np.array_equal(y, h.orc_compute_many(L0.gate_type, L0.down_type, 512, 256, jobs, x))
