// One lane's unit (256 values of one weight row) of each weight type, and its term against a quantised activation unit.
//
// A lane holds one (row, unit) pair of a tile decoded to signed 8-bit words in registers (layout.h: pair idx of a tile
// of nl = 64 U pairs) and takes the activation unit from LDS; each v_dot4 multiplies one word of each. A term is the
// unit's fp32 share of the row sum, with the roundings the CPU oracle's block dot products have (its ORACLE ORDER):
// exact integer sums, then per block (Q8_0) or super-block (Q4_K, IQ3_S) the same fp32 steps.
#pragma once

#include "device_math.h"
#include "layout.h"

namespace c0ven {

// An activation unit (layout.h) as 80 dwords: 64 of codes, the scales at 64, the q8_K sums at 72. It sits in LDS at a
// 16-byte aligned address and is read 16 bytes at a time (ds_read_b128).
struct Act {
  const uint4 *d;
  __device__ __forceinline__ explicit Act(const uint32_t *p) : d((const uint4 *)p) {}
  // Code words 8 i .. 8 i + 7 (the 32 codes of block i).
  __device__ __forceinline__ void q8(int i, uint32_t *w) const {
    const uint4 a = d[2 * i], b = d[2 * i + 1];
    w[0] = a.x, w[1] = a.y, w[2] = a.z, w[3] = a.w, w[4] = b.x, w[5] = b.y, w[6] = b.z, w[7] = b.w;
  }
  __device__ __forceinline__ void scales(float *s) const {
    const uint4 a = d[16], b = d[17];
    s[0] = __uint_as_float(a.x), s[1] = __uint_as_float(a.y), s[2] = __uint_as_float(a.z), s[3] = __uint_as_float(a.w);
    s[4] = __uint_as_float(b.x), s[5] = __uint_as_float(b.y), s[6] = __uint_as_float(b.z), s[7] = __uint_as_float(b.w);
  }
  __device__ __forceinline__ float scale0() const { return __uint_as_float(d[16].x); }
  __device__ __forceinline__ void sums(int *s) const {
    const uint4 a = d[18], b = d[19];
    s[0] = (int)a.x, s[1] = (int)a.y, s[2] = (int)a.z, s[3] = (int)a.w;
    s[4] = (int)b.x, s[5] = (int)b.y, s[6] = (int)b.z, s[7] = (int)b.w;
  }
};

template <typename T>
__device__ __forceinline__ const T *field(const uint8_t *tile, uint32_t base, uint32_t p, uint32_t idx, uint32_t nl) {
  return (const T *)(tile + (uint64_t)base * nl) + (uint64_t)p * nl + idx;
}

// Bytes of g (each at least 1) negated where the matching bit of the four-bit nibble is set, without carries.
__device__ __forceinline__ uint32_t sign4(uint32_t g, uint32_t nib) {
  const uint32_t x = (nib * 0x00204081u) & 0x01010101u;  // byte j = bit j of the nibble
  return (g ^ ((x << 8) - x)) + x;
}

// Q8_0: eight blocks of 32 (vec_dot_q8_0_q8_0). Term: the pairwise sum of (d_w d_a) sumi over the eight blocks.
struct UnitQ8_0 {
  uint32_t q[64];
  float d[8];
  __device__ __forceinline__ void load(const uint8_t *tile, uint32_t idx, uint32_t nl) {
#pragma unroll
    for (int p = 0; p < 16; p++) {
      const uint4 v = *field<uint4>(tile, q8_0t::kQs, p, idx, nl);
      q[4 * p] = v.x, q[4 * p + 1] = v.y, q[4 * p + 2] = v.z, q[4 * p + 3] = v.w;
    }
    const uint4 dv = *field<uint4>(tile, q8_0t::kD, 0, idx, nl);
    const uint32_t w[4] = {dv.x, dv.y, dv.z, dv.w};
#pragma unroll
    for (int b = 0; b < 8; b++) d[b] = h2f((uint16_t)(w[b / 2] >> (16 * (b % 2))));
  }
  __device__ __forceinline__ float term(const Act &a) const {
    float t[8], as[8];
    a.scales(as);
#pragma unroll
    for (int b = 0; b < 8; b++) {
      uint32_t aw[8];
      a.q8(b, aw);
      int s = 0;
#pragma unroll
      for (int i = 0; i < 8; i++) s = dot4(q[8 * b + i], aw[i], s);
      t[b] = __fmul_rn(__fmul_rn(d[b], as[b]), (float)s);
    }
    return __fadd_rn(__fadd_rn(__fadd_rn(t[0], t[1]), __fadd_rn(t[2], t[3])),
                     __fadd_rn(__fadd_rn(t[4], t[5]), __fadd_rn(t[6], t[7])));
  }
};

// Q4_K: eight sub-blocks of 32 with 6-bit scales and minimums (vec_dot_q4_K_q8_K). Term:
// fma(d_w d_a, isum, -((dmin_w d_a) imin)).
struct UnitQ4_K {
  uint32_t lo[32], hi[32];  // the nibbles of qs word w: lo values 64c + 4(w % 8) + 0..3, hi those + 32 (c = w / 8)
  int sc[8], mn[8];
  float d, dmin;
  __device__ __forceinline__ void load(const uint8_t *tile, uint32_t idx, uint32_t nl) {
#pragma unroll
    for (int p = 0; p < 8; p++) {
      const uint4 v = *field<uint4>(tile, q4_kt::kQs, p, idx, nl);
      const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
      for (int i = 0; i < 4; i++) {
        lo[4 * p + i] = w[i] & 0x0f0f0f0fu;
        hi[4 * p + i] = (w[i] >> 4) & 0x0f0f0f0fu;
      }
    }
    uint8_t b[12];
#pragma unroll
    for (int i = 0; i < 3; i++) {
      const uint32_t v = *field<uint32_t>(tile, q4_kt::kScales, i, idx, nl);
#pragma unroll
      for (int j = 0; j < 4; j++) b[4 * i + j] = (uint8_t)(v >> (8 * j));
    }
#pragma unroll
    for (int j = 0; j < 8; j++) {  // get_scale_min_k4
      if (j < 4) {
        sc[j] = b[j] & 63;
        mn[j] = b[j + 4] & 63;
      } else {
        sc[j] = (b[j + 4] & 0xF) | ((b[j - 4] >> 6) << 4);
        mn[j] = (b[j + 4] >> 4) | ((b[j] >> 6) << 4);
      }
    }
    const uint32_t dm = *field<uint32_t>(tile, q4_kt::kDm, 0, idx, nl);
    d = h2f((uint16_t)dm);
    dmin = h2f((uint16_t)(dm >> 16));
  }
  __device__ __forceinline__ float term(const Act &a) const {
    int isum = 0, imin = 0, bs[8];
#pragma unroll
    for (int c = 0; c < 4; c++) {
      uint32_t al[8], ah[8];
      a.q8(2 * c, al);
      a.q8(2 * c + 1, ah);
      int sl = 0, sh = 0;
#pragma unroll
      for (int i = 0; i < 8; i++) {
        sl = dot4(lo[8 * c + i], al[i], sl);
        sh = dot4(hi[8 * c + i], ah[i], sh);
      }
      isum += sc[2 * c] * sl + sc[2 * c + 1] * sh;
    }
    a.sums(bs);
#pragma unroll
    for (int j = 0; j < 8; j++) imin += mn[j] * bs[j];
    const float ad = a.scale0();
    const float dd = __fmul_rn(d, ad), dm = __fmul_rn(dmin, ad);
    const float pm = __fmul_rn(dm, (float)imin);
    return __builtin_fmaf(dd, (float)isum, -pm);
  }
};

// IQ3_S: 64 groups of 4 from the 512-entry grid, signs stored plainly, 4-bit scales (vec_dot_iq3_s_q8_K). Term:
// (d_w d_a) sum_ib (1 + 2 s_ib) sumi_ib.
struct UnitIQ3_S {
  uint32_t w[64];  // group k's four values 4k..4k+3, signed
  int ls[8];
  float d;
  __device__ __forceinline__ void load(const uint8_t *tile, uint32_t idx, uint32_t nl, const uint32_t *grid) {
    uint32_t qs[16], sg[8];
#pragma unroll
    for (int p = 0; p < 4; p++) {
      const uint4 v = *field<uint4>(tile, iq3_st::kQs, p, idx, nl);
      qs[4 * p] = v.x, qs[4 * p + 1] = v.y, qs[4 * p + 2] = v.z, qs[4 * p + 3] = v.w;
    }
#pragma unroll
    for (int p = 0; p < 2; p++) {
      const uint4 v = *field<uint4>(tile, iq3_st::kSigns, p, idx, nl);
      sg[4 * p] = v.x, sg[4 * p + 1] = v.y, sg[4 * p + 2] = v.z, sg[4 * p + 3] = v.w;
    }
    const uint32_t qh[2] = {*field<uint32_t>(tile, iq3_st::kQh, 0, idx, nl), *field<uint32_t>(tile, iq3_st::kQh, 1, idx, nl)};
    const uint32_t sc = *field<uint32_t>(tile, iq3_st::kScales, 0, idx, nl);
    d = h2f(*field<uint16_t>(tile, iq3_st::kD, 0, idx, nl));
#pragma unroll
    for (int ib = 0; ib < 8; ib++) ls[ib] = 1 + 2 * (int)((sc >> (4 * ib)) & 15u);
#pragma unroll
    for (int k = 0; k < 64; k++) {
      const uint32_t ix = ((qs[k / 4] >> (8 * (k % 4))) & 0xffu) | (((qh[k / 32] >> (k % 32)) & 1u) << 8);
      const uint32_t g = grid[ix];
      w[k] = sign4(g, (sg[k / 8] >> (4 * (k % 8))) & 15u);
    }
  }
  __device__ __forceinline__ float term(const Act &a) const {
    int bsum = 0;
#pragma unroll
    for (int ib = 0; ib < 8; ib++) {
      uint32_t aw[8];
      a.q8(ib, aw);
      int s = 0;
#pragma unroll
      for (int k = 0; k < 8; k++) s = dot4(w[8 * ib + k], aw[k], s);
      bsum += ls[ib] * s;
    }
    return __fmul_rn(__fmul_rn(d, a.scale0()), (float)bsum);
  }
};

// IQ3_XXS: eight sub-blocks of 32, each eight grid groups of 4 (iq3xxs_grid, 256 entries in LDS) with signs in fours
// of seven bits, the eighth the parity (multirow.cpp:126-176, vec_dot_iq3_xxs_q8_K). Term: 0.25 ((d_w d_a) isum),
// isum = sum over sub-blocks of (2 s + 1) times the sub-block's exact dot; the factor 0.25 is a power of two.
struct UnitIQ3_XXS {
  uint32_t w[64];  // group k's four values 4k..4k+3, signed
  int ls[8];
  float d;
  __device__ __forceinline__ void load(const uint8_t *tile, uint32_t idx, uint32_t nl, const uint32_t *grid) {
    uint32_t qs[16], ss[8];
#pragma unroll
    for (int p = 0; p < 4; p++) {
      const uint4 v = *field<uint4>(tile, iq3_xxst::kQs, p, idx, nl);
      qs[4 * p] = v.x, qs[4 * p + 1] = v.y, qs[4 * p + 2] = v.z, qs[4 * p + 3] = v.w;
    }
#pragma unroll
    for (int p = 0; p < 2; p++) {
      const uint4 v = *field<uint4>(tile, iq3_xxst::kSs, p, idx, nl);
      ss[4 * p] = v.x, ss[4 * p + 1] = v.y, ss[4 * p + 2] = v.z, ss[4 * p + 3] = v.w;
    }
    d = h2f(*field<uint16_t>(tile, iq3_xxst::kD, 0, idx, nl));
#pragma unroll
    for (int b = 0; b < 8; b++) ls[b] = 2 * (int)(ss[b] >> 28) + 1;
#pragma unroll
    for (int k = 0; k < 64; k++) {  // group k: sub-block k / 8, sign group (k % 8) / 2, its half k % 2
      const uint32_t s7 = (ss[k / 8] >> (7 * ((k % 8) / 2))) & 127u;
      const uint32_t sb = s7 | ((uint32_t)(__popc(s7) & 1) << 7);
      w[k] = sign4(grid[(qs[k / 4] >> (8 * (k % 4))) & 0xffu], (sb >> (4 * (k % 2))) & 15u);
    }
  }
  __device__ __forceinline__ float term(const Act &a) const {
    int bsum = 0;
#pragma unroll
    for (int ib = 0; ib < 8; ib++) {
      uint32_t aw[8];
      a.q8(ib, aw);
      int s = 0;
#pragma unroll
      for (int k = 0; k < 8; k++) s = dot4(w[8 * ib + k], aw[k], s);
      bsum += ls[ib] * s;
    }
    return __fmul_rn(0.25f, __fmul_rn(__fmul_rn(d, a.scale0()), (float)bsum));
  }
};

// IQ2_S: eight sub-blocks of 32, each four groups of 8 values from iq2s_grid (1024 entries of 8 bytes, in LDS as
// word pairs) with a 10-bit index and 8 sign bits; a 4-bit scale for each half sub-block (multirow.cpp:68-124,
// vec_dot_iq2_s_q8_K). Term: 0.125 ((d_w d_a) isum), isum = sum over half sub-blocks of (2 s + 1) times the exact dot.
struct UnitIQ2_S {
  uint32_t w[64];  // values 4k..4k+3, signed
  int ls[16];      // half sub-block h: values 16 h .. 16 h + 15
  float d;
  __device__ __forceinline__ void load(const uint8_t *tile, uint32_t idx, uint32_t nl, const uint32_t *grid) {
    uint32_t qs[8], sg[8];
#pragma unroll
    for (int p = 0; p < 2; p++) {
      const uint4 v = *field<uint4>(tile, iq2_st::kQs, p, idx, nl), u = *field<uint4>(tile, iq2_st::kSigns, p, idx, nl);
      qs[4 * p] = v.x, qs[4 * p + 1] = v.y, qs[4 * p + 2] = v.z, qs[4 * p + 3] = v.w;
      sg[4 * p] = u.x, sg[4 * p + 1] = u.y, sg[4 * p + 2] = u.z, sg[4 * p + 3] = u.w;
    }
    const uint2 qh = *field<uint2>(tile, iq2_st::kQh, 0, idx, nl), sc = *field<uint2>(tile, iq2_st::kScales, 0, idx, nl);
    d = h2f(*field<uint16_t>(tile, iq2_st::kD, 0, idx, nl));
#pragma unroll
    for (int h = 0; h < 16; h++) ls[h] = 2 * (int)((((h < 8) ? sc.x : sc.y) >> (4 * (h % 8))) & 15u) + 1;
#pragma unroll
    for (int gi = 0; gi < 32; gi++) {  // group gi = 4 b + g: sub-block b, values 8 g .. 8 g + 7 of it
      const uint32_t b = gi / 4, g = gi % 4;
      const uint32_t hbits = (((b < 4) ? qh.x : qh.y) >> (8 * (b % 4) + 2 * g)) & 3u;
      const uint32_t ix = ((qs[gi / 4] >> (8 * (gi % 4))) & 0xffu) | (hbits << 8);
      const uint32_t sb = (sg[gi / 4] >> (8 * (gi % 4))) & 0xffu;
      w[2 * gi] = sign4(grid[2 * ix], sb & 15u);
      w[2 * gi + 1] = sign4(grid[2 * ix + 1], sb >> 4);
    }
  }
  __device__ __forceinline__ float term(const Act &a) const {
    int isum = 0;
#pragma unroll
    for (int ib = 0; ib < 8; ib++) {
      uint32_t aw[8];
      a.q8(ib, aw);
      int s0 = 0, s1 = 0;
#pragma unroll
      for (int k = 0; k < 4; k++) s0 = dot4(w[8 * ib + k], aw[k], s0);
#pragma unroll
      for (int k = 4; k < 8; k++) s1 = dot4(w[8 * ib + k], aw[k], s1);
      isum += ls[2 * ib] * s0 + ls[2 * ib + 1] * s1;
    }
    return __fmul_rn(0.125f, __fmul_rn(__fmul_rn(d, a.scale0()), (float)isum));
  }
};

// kvalues_iq4nl (ggml-common.h; -127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113, whose
// sha256 docs/spec/QUANT_FORMATS.md:547 records) as four little-endian words of table bytes 0-3, 4-7, 8-11, 12-15.
constexpr uint32_t kIq4nlW0 = 0xBFAD9881u, kIq4nlW1 = 0xF6EADDCFu, kIq4nlW2 = 0x26190D01u, kIq4nlW3 = 0x71594535u;

// Four nibbles (the bytes of n, each 0..15) to their four codebook values (signed bytes): two byte permutes pick from
// table bytes 0-7 and 8-15, bit 3 of each nibble chooses between them.
__device__ __forceinline__ uint32_t iq4nl_lookup(uint32_t n) {
  const uint32_t sel = n & 0x07070707u;
  const uint32_t lo = __builtin_amdgcn_perm(kIq4nlW1, kIq4nlW0, sel), hi = __builtin_amdgcn_perm(kIq4nlW3, kIq4nlW2, sel);
  const uint32_t b = (n >> 3) & 0x01010101u, m = (b << 8) - b;  // 0xff where the nibble is 8..15
  return (hi & m) | (lo & ~m);
}

// The four 2-bit codes of byte x (value j at bits 2 j) as four signed bytes q - 1 (Q2_0's -1, 0, 1, 2).
__device__ __forceinline__ uint32_t q2_spread(uint32_t x) {
  const uint32_t s = (x | (x << 6) | (x << 12) | (x << 18)) & 0x03030303u;
  return ((s | 0x80808080u) - 0x01010101u) ^ 0x80808080u;  // per byte (0x80 + q) - 1, no borrows, back to q - 1
}

// IQ4_NL: eight blocks of 32, y = d kvalues[nibble] (dequantize_row_iq4_nl; vec_dot_iq4_nl_q8_0 against q8_0). The
// codes decode to the signed bytes a Q8_0 block holds, so the term is UnitQ8_0's: pairwise over the eight blocks of
// (d_w d_a) sumi.
struct UnitIQ4_NL : UnitQ8_0 {
  __device__ __forceinline__ void load(const uint8_t *tile, uint32_t idx, uint32_t nl) {
#pragma unroll
    for (int p = 0; p < 8; p++) {  // block p: values 0-15 the low nibbles of its 16 bytes, 16-31 the high ones
      const uint4 v = *field<uint4>(tile, iq4_nlt::kQs, p, idx, nl);
      const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
      for (int i = 0; i < 4; i++) {
        q[8 * p + i] = iq4nl_lookup(w[i] & 0x0f0f0f0fu);
        q[8 * p + 4 + i] = iq4nl_lookup((w[i] >> 4) & 0x0f0f0f0fu);
      }
    }
    const uint4 dv = *field<uint4>(tile, iq4_nlt::kD, 0, idx, nl);
    const uint32_t w[4] = {dv.x, dv.y, dv.z, dv.w};
#pragma unroll
    for (int b = 0; b < 8; b++) d[b] = h2f((uint16_t)(w[b / 2] >> (16 * (b % 2))));
  }
};

// Q2_0: four blocks of 64 with one f16 scale, y = (q - 1) d (dequantize_row_q2_0), against q8_0 blocks of 32: each
// half block is a Q8_0-like block of codes q - 1 with the block's d, so the term is UnitQ8_0's over the eight halves.
struct UnitQ2_0 : UnitQ8_0 {
  __device__ __forceinline__ void load(const uint8_t *tile, uint32_t idx, uint32_t nl) {
#pragma unroll
    for (int p = 0; p < 4; p++) {  // block p: half 2 p is bytes 0-7, half 2 p + 1 bytes 8-15, four codes a byte
      const uint4 v = *field<uint4>(tile, q2_0t::kQs, p, idx, nl);
      const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
      for (int i = 0; i < 16; i++) q[16 * p + i] = q2_spread((w[i / 4] >> (8 * (i % 4))) & 0xffu);
    }
    const uint2 dv = *field<uint2>(tile, q2_0t::kD, 0, idx, nl);
    const uint32_t w[2] = {dv.x, dv.y};
#pragma unroll
    for (int h = 0; h < 8; h++) d[h] = h2f((uint16_t)(w[h / 4] >> (16 * ((h / 2) % 2))));
  }
};

// IQ4_XS: eight sub-blocks of 32 with a 6-bit scale ls (4 bits in scales_l, 2 in scales_h), values d (ls - 32)
// kvalues[nibble] (QUANT_FORMATS.md:213-232; vec_dot_iq4_xs_q8_K). Term: (d_w d_a) isum, isum = sum over sub-blocks
// of (ls - 32) times the sub-block's exact dot.
struct UnitIQ4_XS {
  uint32_t q[64];  // sub-block p: words 8 p .. 8 p + 3 values 0-15 (low nibbles), 8 p + 4 .. values 16-31
  int ls[8];
  float d;
  __device__ __forceinline__ void load(const uint8_t *tile, uint32_t idx, uint32_t nl) {
#pragma unroll
    for (int p = 0; p < 8; p++) {
      const uint4 v = *field<uint4>(tile, iq4_xst::kQs, p, idx, nl);
      const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
      for (int i = 0; i < 4; i++) {
        q[8 * p + i] = iq4nl_lookup(w[i] & 0x0f0f0f0fu);
        q[8 * p + 4 + i] = iq4nl_lookup((w[i] >> 4) & 0x0f0f0f0fu);
      }
    }
    const uint2 m = *field<uint2>(tile, iq4_xst::kMeta, 0, idx, nl);  // d | scales_h << 16, scales_l
    d = h2f((uint16_t)m.x);
#pragma unroll
    for (int b = 0; b < 8; b++)
      ls[b] = (int)(((m.y >> (4 * b)) & 15u) | (((m.x >> (16 + 2 * b)) & 3u) << 4)) - 32;
  }
  __device__ __forceinline__ float term(const Act &a) const {
    int bsum = 0;
#pragma unroll
    for (int ib = 0; ib < 8; ib++) {
      uint32_t aw[8];
      a.q8(ib, aw);
      int s = 0;
#pragma unroll
      for (int k = 0; k < 8; k++) s = dot4(q[8 * ib + k], aw[k], s);
      bsum += ls[ib] * s;
    }
    return __fmul_rn(__fmul_rn(d, a.scale0()), (float)bsum);
  }
};

// Q5_K: Q4_K with a fifth bit per value from qh (bit k of byte l is bit 4 of value 32 k + l; QUANT_FORMATS.md:401-417,
// vec_dot_q5_K_q8_K). The codes are 0..31 and the term is Q4_K's.
struct UnitQ5_K : UnitQ4_K {
  __device__ __forceinline__ void load(const uint8_t *tile, uint32_t idx, uint32_t nl) {
    uint32_t qh[8];
#pragma unroll
    for (int p = 0; p < 2; p++) {
      const uint4 v = *field<uint4>(tile, q5_kt::kQh, p, idx, nl);
      qh[4 * p] = v.x, qh[4 * p + 1] = v.y, qh[4 * p + 2] = v.z, qh[4 * p + 3] = v.w;
    }
#pragma unroll
    for (int p = 0; p < 8; p++) {
      const uint4 v = *field<uint4>(tile, q5_kt::kQs, p, idx, nl);
      const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
      for (int i = 0; i < 4; i++) {  // word 4 p + i: chunk c = p / 2, bytes 4 (w % 8) .. of it
        const uint32_t wi = 4 * p + i, c = wi / 8, h = qh[wi % 8];
        lo[wi] = (w[i] & 0x0f0f0f0fu) | (((h >> (2 * c)) & 0x01010101u) << 4);
        hi[wi] = ((w[i] >> 4) & 0x0f0f0f0fu) | (((h >> (2 * c + 1)) & 0x01010101u) << 4);
      }
    }
    uint8_t b[12];
#pragma unroll
    for (int i = 0; i < 3; i++) {
      const uint32_t v = *field<uint32_t>(tile, q5_kt::kScales, i, idx, nl);
#pragma unroll
      for (int j = 0; j < 4; j++) b[4 * i + j] = (uint8_t)(v >> (8 * j));
    }
#pragma unroll
    for (int j = 0; j < 8; j++) {  // get_scale_min_k4
      if (j < 4) {
        sc[j] = b[j] & 63;
        mn[j] = b[j + 4] & 63;
      } else {
        sc[j] = (b[j + 4] & 0xF) | ((b[j - 4] >> 6) << 4);
        mn[j] = (b[j + 4] >> 4) | ((b[j] >> 6) << 4);
      }
    }
    const uint32_t dm = *field<uint32_t>(tile, q5_kt::kDm, 0, idx, nl);
    d = h2f((uint16_t)dm);
    dmin = h2f((uint16_t)(dm >> 16));
  }
};

// Four bytes of six-bit codes (0..63) less 32, as signed bytes: per byte (0x80 + c) - 32 has no borrow, then back.
__device__ __forceinline__ uint32_t sub32_bytes(uint32_t c) { return ((c | 0x80808080u) - 0x20202020u) ^ 0x80808080u; }

// The word (values 4 k .. 4 k + 3) of a Q6_K super-block from its ql and qh words (QUANT_FORMATS.md:419-445): value
// v = 128 h + 32 j + l takes the nibble 4 (j / 2) of ql byte 64 h + 32 (j % 2) + l and bits 2 j of qh byte 32 h + l.
__device__ __forceinline__ uint32_t q6k_word(const uint32_t *ql, const uint32_t *qh, uint32_t k) {
  const uint32_t v = 4 * k, h = v / 128, j = (v % 128) / 32, l = v % 32;
  const uint32_t lw = ql[(64 * h + 32 * (j % 2) + l) / 4], hw = qh[(32 * h + l) / 4];
  return sub32_bytes(((lw >> (4 * (j / 2))) & 0x0f0f0f0fu) | (((hw >> (2 * j)) & 0x03030303u) << 4));
}

// Q6_K: sixteen sub-blocks of 16 with signed 8-bit scales, values d sc (q - 32) (vec_dot_q6_K_q8_K). Term:
// (d_w d_a) isum, isum = sum over sub-blocks of sc times the sub-block's exact dot.
struct UnitQ6_K {
  uint32_t w[64];  // values 4 k .. 4 k + 3, signed
  int sc[16];
  float d;
  __device__ __forceinline__ void load(const uint8_t *tile, uint32_t idx, uint32_t nl) {
    uint32_t ql[32], qh[16];
#pragma unroll
    for (int p = 0; p < 8; p++) {
      const uint4 v = *field<uint4>(tile, q6_kt::kQl, p, idx, nl);
      ql[4 * p] = v.x, ql[4 * p + 1] = v.y, ql[4 * p + 2] = v.z, ql[4 * p + 3] = v.w;
    }
#pragma unroll
    for (int p = 0; p < 4; p++) {
      const uint4 v = *field<uint4>(tile, q6_kt::kQh, p, idx, nl);
      qh[4 * p] = v.x, qh[4 * p + 1] = v.y, qh[4 * p + 2] = v.z, qh[4 * p + 3] = v.w;
    }
    const uint4 s = *field<uint4>(tile, q6_kt::kScales, 0, idx, nl);
    const uint32_t sw[4] = {s.x, s.y, s.z, s.w};
#pragma unroll
    for (int i = 0; i < 16; i++) sc[i] = (int)(int8_t)(sw[i / 4] >> (8 * (i % 4)));
    d = h2f(*field<uint16_t>(tile, q6_kt::kD, 0, idx, nl));
#pragma unroll
    for (uint32_t k = 0; k < 64; k++) w[k] = q6k_word(ql, qh, k);
  }
  __device__ __forceinline__ float term(const Act &a) const {
    int isum = 0;
#pragma unroll
    for (int ib = 0; ib < 8; ib++) {
      uint32_t aw[8];
      a.q8(ib, aw);
      int s0 = 0, s1 = 0;
#pragma unroll
      for (int k = 0; k < 4; k++) s0 = dot4(w[8 * ib + k], aw[k], s0);
#pragma unroll
      for (int k = 4; k < 8; k++) s1 = dot4(w[8 * ib + k], aw[k], s1);
      isum += sc[2 * ib] * s0 + sc[2 * ib + 1] * s1;
    }
    return __fmul_rn(__fmul_rn(d, a.scale0()), (float)isum);
  }
};

// IQ4_NL and Q2_0 as UnitQ8_0 with the decode split from the loads: load_raw issues a unit's loads (IQ4_NL its 32
// nibble words into q[0..31]; Q2_0 its 16 code words into q[0..15]; the f16 scale words into dw), and widen, once
// they have arrived, decodes them in place exactly as UnitIQ4_NL::load / UnitQ2_0::load do. A caller that takes
// the type at run time gives each type its own branch of load_raw, wait, widen and terms, so that no two types'
// registers are live together.
template <uint32_t kT>
struct UnitQ8Split : UnitQ8_0 {
  static_assert(kT == QT_IQ4_NL || kT == QT_Q2_0, "UnitQ8Split: IQ4_NL or Q2_0");
  static constexpr uint32_t kPieces = kT == QT_IQ4_NL ? 8 : 4;  // 16-byte pieces of codes
  uint32_t dw[4];
  __device__ __forceinline__ void load_raw(const uint8_t *tile, uint32_t idx, uint32_t nl) {
#pragma unroll
    for (uint32_t p = 0; p < kPieces; p++) {
      const uint4 v = *field<uint4>(tile, 0, p, idx, nl);
      q[4 * p] = v.x, q[4 * p + 1] = v.y, q[4 * p + 2] = v.z, q[4 * p + 3] = v.w;
    }
    if constexpr (kT == QT_Q2_0) {
      const uint2 v = *field<uint2>(tile, q2_0t::kD, 0, idx, nl);
      dw[0] = v.x, dw[1] = v.y;
    } else {
      const uint4 v = *field<uint4>(tile, iq4_nlt::kD, 0, idx, nl);
      dw[0] = v.x, dw[1] = v.y, dw[2] = v.z, dw[3] = v.w;
    }
  }
  __device__ __forceinline__ void widen() {
#pragma unroll
    for (int p = (int)kPieces - 1; p >= 0; p--) {  // descending: piece p's words move to 8p.. or 16p.., never onto a
      const uint32_t w[4] = {q[4 * p], q[4 * p + 1], q[4 * p + 2], q[4 * p + 3]};  // piece not yet read
      if constexpr (kT == QT_IQ4_NL) {
#pragma unroll
        for (int i = 0; i < 4; i++) {
          q[8 * p + i] = iq4nl_lookup(w[i] & 0x0f0f0f0fu);
          q[8 * p + 4 + i] = iq4nl_lookup((w[i] >> 4) & 0x0f0f0f0fu);
        }
      } else {
#pragma unroll
        for (int i = 0; i < 16; i++) q[16 * p + i] = q2_spread((w[i / 4] >> (8 * (i % 4))) & 0xffu);
      }
    }
#pragma unroll
    for (int b = 0; b < 8; b++)
      d[b] = h2f((uint16_t)(kT == QT_Q2_0 ? dw[b / 4] >> (16 * ((b / 2) % 2)) : dw[b / 2] >> (16 * (b % 2))));
  }
};

}  // namespace c0ven
