// Q4_K weights against a group's activations on the matrix cores: 16 weight rows x 16 token columns x one unit (256
// values) per set of v_mfma_i32_16x16x64_i8 (the codes) and v_mfma_i32_16x16x32_i8 (the minimum part), with the same
// integers and fp32 steps as UnitQ4_K::term (units.h).
//
// Operand layout (one wave): lane l holds A row l % 16 and B column l % 16, bytes 8 g .. 8 g + 7 of each 32-value
// block, g = l / 16; the result D[row][col] sits in lane 16 (row / 4) + col as element row % 4. Here A is the weights
// (row = weight row) and B the activations (col = token), so lane l ends with rows 4 g + i (i < 4) of token l % 16.
//
// Exactness: Q4_K's sub-block scale sc_j (6 bits) is split as 8 hi + lo (3 bits each) and folded into the codes
// (q <= 15 times at most 7 fits a byte), so one accumulating chain gives sum_j (q lo_j) . a and another
// sum_j (q hi_j) . a: isum = 8 D_hi + D_lo, exactly the integer of the CPU path. The minimum part
// imin = sum_j mn_j bsum_j takes two more: bsum_j = 64 hi + lo (hi in [-64, 63], lo in [0, 63]).
#pragma once

#include "device_math.h"
#include "layout.h"

namespace c0ven {

typedef int v4i_t __attribute__((ext_vector_type(4)));
typedef unsigned short u16x2_t __attribute__((ext_vector_type(2)));

// Each byte of w (at most 15) times k (at most 7, in both 16-bit halves of kk): two 16-bit products per word, no
// carry between bytes.
__device__ __forceinline__ uint32_t mul_bytes(uint32_t w, uint32_t kk) {
  return __builtin_bit_cast(uint32_t, __builtin_bit_cast(u16x2_t, w) * __builtin_bit_cast(u16x2_t, kk));
}
__device__ __forceinline__ long pack2(uint32_t lo, uint32_t hi) { return (long)(((uint64_t)hi << 32) | lo); }

// One lane's raw bytes of a 16-row x 1-unit Q4_K tile: its A row's qs (8 bytes of each 64-value chunk) and scales,
// and the d|dmin words of its four D rows.
struct Q4kRaw {
  uint2 qs[4];
  uint32_t sc[3], dm[4];
  // Rows row0 .. row0 + 15 (row0 a multiple of 16) of the matrix at mat (U units a row), unit u: the codes (four
  // 8-byte loads) and the scales with d|dmin (four loads), which load_qs / load_meta issue separately.
  __device__ __forceinline__ void load(const uint8_t *mat, uint32_t U, uint32_t row0, uint32_t u, uint32_t lane) {
    load_qs(mat, U, row0, u, lane);
    load_meta(mat, U, row0, u, lane);
  }
  // Addresses as a wave-uniform pointer (tile, field, unit) plus a 32-bit lane offset, so that each load is one
  // global load on a scalar base with no per-load vector address arithmetic.
  __device__ __forceinline__ void load_qs(const uint8_t *mat, uint32_t U, uint32_t row0, uint32_t u, uint32_t lane) {
    const uint32_t g = lane / 16, nl = kTileRows * U;
    const uint8_t *tile = mat + (uint64_t)(row0 / kTileRows) * tile_bytes(QT_Q4_K, U) + (uint64_t)u * kTileRows * 16;
    const uint32_t lo = (g / 2) * nl * 16 + ((row0 % kTileRows) + lane % 16) * 16 + 8 * (g % 2);
#pragma unroll
    for (uint32_t c = 0; c < 4; c++) qs[c] = *(const uint2 *)(tile + (uint64_t)(q4_kt::kQs / 16 + 2 * c) * nl * 16 + lo);
  }
  __device__ __forceinline__ void load_meta(const uint8_t *mat, uint32_t U, uint32_t row0, uint32_t u, uint32_t lane) {
    const uint32_t g = lane / 16, nl = kTileRows * U;
    const uint8_t *tile = mat + (uint64_t)(row0 / kTileRows) * tile_bytes(QT_Q4_K, U) + (uint64_t)u * kTileRows * 4;
    const uint32_t ls = ((row0 % kTileRows) + lane % 16) * 4, ld = ((row0 % kTileRows) + 4 * g) * 4;
#pragma unroll
    for (uint32_t i = 0; i < 3; i++) sc[i] = *(const uint32_t *)(tile + (uint64_t)(q4_kt::kScales + 4 * i) * nl + ls);
    // The four D rows' words are consecutive pairs (16-byte aligned: 4 g + row0 % 64 is a multiple of 4): one load.
    const uint4 v = *(const uint4 *)(tile + (uint64_t)q4_kt::kDm * nl + ld);
    dm[0] = v.x, dm[1] = v.y, dm[2] = v.z, dm[3] = v.w;
  }
};

// {byte b of v, 0, byte b of v, 0}: a byte as the two 16-bit halves of a packed multiplier.
__device__ __forceinline__ uint32_t bcast_byte(uint32_t v, uint32_t b) {
  return __builtin_amdgcn_perm(0u, v, 0x0c000c00u | (b << 16) | b);
}

// The A operands of one tile-unit and its D rows' scales. The six-bit scales and minima of the eight blocks are
// unpacked four to a word (get_scale_min_k4 on all four bytes at once): blocks 0-3 are the low six bits of bytes
// 0-3 (scales) and 4-7 (minima); blocks 4-7 take four bits from bytes 8-11 and their top two from the top bits of
// bytes 0-3 (scales) and 4-7 (minima).
struct Q4kA {
  v4i_t lo[4], hi[4];  // chain step c: blocks 2 c (elements 0-1) and 2 c + 1 (elements 2-3), as join2 packs them
  long mn;
  float d[4], dmin[4];
  // kHalfMin: mn as the f16 operand of the prefill form (q4k_terms_p) rather than the int8 one (q4k_terms_v).
  template <bool kHalfMin = false>
  __device__ __forceinline__ void decode(const Q4kRaw &r, uint32_t lane) {
    const uint32_t w0 = r.sc[0], w1 = r.sc[1], w2 = r.sc[2];
    const uint32_t sc03 = w0 & 0x3f3f3f3fu, sc47 = (w2 & 0x0f0f0f0fu) | ((w0 >> 2) & 0x30303030u);
    const uint32_t m03 = w1 & 0x3f3f3f3fu, m47 = ((w2 >> 4) & 0x0f0f0f0fu) | ((w1 >> 2) & 0x30303030u);
    // Each scale split 8 hi + lo (three bits each), four blocks a word.
    const uint32_t slo[2] = {sc03 & 0x07070707u, sc47 & 0x07070707u};
    const uint32_t shi[2] = {(sc03 >> 3) & 0x07070707u, (sc47 >> 3) & 0x07070707u};
#pragma unroll
    for (int c = 0; c < 4; c++) {
      const uint32_t w0q = r.qs[c].x, w1q = r.qs[c].y;
      const uint32_t l0 = w0q & 0x0f0f0f0fu, l1 = w1q & 0x0f0f0f0fu;
      const uint32_t h0 = (w0q >> 4) & 0x0f0f0f0fu, h1 = (w1q >> 4) & 0x0f0f0f0fu;
      const uint32_t bl = (2 * c) % 4, bh = (2 * c + 1) % 4, hw = c / 2;  // blocks 2 c, 2 c + 1: bytes, word
      const uint32_t kl_lo = bcast_byte(slo[hw], bl), kl_hi = bcast_byte(shi[hw], bl);
      const uint32_t kh_lo = bcast_byte(slo[hw], bh), kh_hi = bcast_byte(shi[hw], bh);
      lo[c] = v4i_t{(int)mul_bytes(l0, kl_lo), (int)mul_bytes(l1, kl_lo), (int)mul_bytes(h0, kh_lo), (int)mul_bytes(h1, kh_lo)};
      hi[c] = v4i_t{(int)mul_bytes(l0, kl_hi), (int)mul_bytes(l1, kl_hi), (int)mul_bytes(h0, kh_hi), (int)mul_bytes(h1, kh_hi)};
    }
    if constexpr (kHalfMin) {
      // The A operand of v_mfma_f32_16x16x16_f16 against kActSplitH's split sums: k = 0-7 and 8-15 both the minima
      // 0-7, so lane group g takes minima 4 (g % 2) .. + 3 as f16 (exact: at most 63).
      const uint32_t m = (lane / 16) % 2 ? m47 : m03;
      const auto h01 = __builtin_amdgcn_cvt_pkrtz((float)(m & 0xffu), (float)((m >> 8) & 0xffu));
      const auto h23 = __builtin_amdgcn_cvt_pkrtz((float)((m >> 16) & 0xffu), (float)(m >> 24));
      mn = pack2(__builtin_bit_cast(uint32_t, h01), __builtin_bit_cast(uint32_t, h23));
    } else {
      mn = lane < 16 ? pack2(m03, m47) : 0;
    }
#pragma unroll
    for (int i = 0; i < 4; i++) d[i] = h2f((uint16_t)r.dm[i]), dmin[i] = h2f((uint16_t)(r.dm[i] >> 16));
  }
};

// One lane's B operands of an activation unit (token l % 16 of the group, clamped to the last real one): the codes of
// each 32-value block, the block sums split for the minimum part, and the unit's scale.
struct ActB {
  long q[8], bh, bl;
  float ad;
  __device__ __forceinline__ void load(const uint8_t *unit, uint32_t lane) {
    const uint32_t g = lane / 16;
#pragma unroll
    for (int s = 0; s < 8; s++) q[s] = *(const long *)(unit + 32 * s + 8 * g);
    split_sums(unit, g);
    ad = *(const float *)(unit + kActScales);
  }
  // The same, with the sums' split already in the unit's padding (at kActSplit, written by put_split).
  __device__ __forceinline__ void load_presplit(const uint8_t *unit, uint32_t lane) {
    const uint32_t g = lane / 16;
#pragma unroll
    for (int s = 0; s < 8; s++) q[s] = *(const long *)(unit + 32 * s + 8 * g);
    const uint4 v = *(const uint4 *)(unit + kActSplit);
    bh = g == 0 ? pack2(v.x, v.y) : 0;
    bl = g == 0 ? pack2(v.z, v.w) : 0;
    ad = *(const float *)(unit + kActScales);
  }
  // Writes a unit's split sums (hi bytes, then lo bytes) into its LDS padding at kActSplit.
  __device__ static __forceinline__ void put_split(uint8_t *unit) {
    uint32_t h[2], l[2];
    split_words(unit, h, l);
    *(uint4 *)(unit + kActSplit) = make_uint4(h[0], h[1], l[0], l[1]);
  }
  __device__ static __forceinline__ void split_words(const uint8_t *unit, uint32_t h[2], uint32_t l[2]) {
    const uint4 a = *(const uint4 *)(unit + kActSums), c = *(const uint4 *)(unit + kActSums + 16);
    const int bs[8] = {(int)a.x, (int)a.y, (int)a.z, (int)a.w, (int)c.x, (int)c.y, (int)c.z, (int)c.w};
    h[0] = h[1] = l[0] = l[1] = 0u;
#pragma unroll
    for (int j = 0; j < 8; j++) {
      h[j / 4] |= ((uint32_t)(bs[j] >> 6) & 0xffu) << (8 * (j % 4));
      l[j / 4] |= ((uint32_t)bs[j] & 63u) << (8 * (j % 4));
    }
  }
  __device__ __forceinline__ void split_sums(const uint8_t *unit, uint32_t g) {
    uint32_t h[2], l[2];
    split_words(unit, h, l);
    bh = g == 0 ? pack2(h[0], h[1]) : 0;
    bl = g == 0 ? pack2(l[0], l[1]) : 0;
  }
};

// Two 8-byte operand pieces as one 16-byte operand of v_mfma_i32_16x16x64_i8.
__device__ __forceinline__ v4i_t join2(long x, long y) {
  return v4i_t{(int)x, (int)((uint64_t)x >> 32), (int)y, (int)((uint64_t)y >> 32)};
}

// The unit's terms t[i] (rows 4 g + i, token l % 16): fma(d ad, isum, -((dmin ad) imin)) as UnitQ4_K::term.
// The code chains take two blocks per v_mfma_i32_16x16x64_i8 (blocks 2 c and 2 c + 1: a lane's eight bytes of each,
// in A and in B alike, so every A byte still meets its own activation byte; the sum over K is the same integer).
// bq[c]: the lane's B operand of chain step c; bh, bl: the split block sums (lanes < 16); ad: the unit's scale.
__device__ __forceinline__ void q4k_terms_v(const Q4kA &a, const v4i_t bq[4], long bh, long bl, float ad, float t[4]) {
  v4i_t dlo = {0, 0, 0, 0}, dhi = {0, 0, 0, 0};
#pragma unroll
  for (int c = 0; c < 4; c++) {
    dlo = __builtin_amdgcn_mfma_i32_16x16x64_i8(a.lo[c], bq[c], dlo, 0, 0, 0);
    dhi = __builtin_amdgcn_mfma_i32_16x16x64_i8(a.hi[c], bq[c], dhi, 0, 0, 0);
  }
  const v4i_t mh = __builtin_amdgcn_mfma_i32_16x16x32_i8(a.mn, bh, v4i_t{0, 0, 0, 0}, 0, 0, 0);
  const v4i_t ml = __builtin_amdgcn_mfma_i32_16x16x32_i8(a.mn, bl, v4i_t{0, 0, 0, 0}, 0, 0, 0);
#pragma unroll
  for (int i = 0; i < 4; i++) {
    const int isum = 8 * dhi[i] + dlo[i], imin = 64 * mh[i] + ml[i];
    const float dd = __fmul_rn(a.d[i], ad), dm = __fmul_rn(a.dmin[i], ad);
    const float pm = __fmul_rn(dm, (float)imin);
    t[i] = __builtin_fmaf(dd, (float)isum, -pm);
  }
}

__device__ __forceinline__ void q4k_terms(const Q4kA &a, const ActB &b, float t[4]) {
  v4i_t bq[4];
#pragma unroll
  for (int c = 0; c < 4; c++) bq[c] = join2(b.q[2 * c], b.q[2 * c + 1]);
  q4k_terms_v(a, bq, b.bh, b.bl, b.ad, t);
}

// A prefill activation unit's B operands (codes in the mfma_code_off order, split sums as f16 at kActSplitH): four
// 16-byte reads for the code chains, one 8-byte read for the minimum part.
struct ActBP {
  v4i_t q[4];
  long bm;
  float ad;
  __device__ __forceinline__ void load(const uint8_t *unit, uint32_t lane) {
    const uint32_t g = lane / 16;
#pragma unroll
    for (int c = 0; c < 4; c++) q[c] = *(const v4i_t *)(unit + 64 * c + 16 * g);
    bm = *(const long *)(unit + kActSplitH + 8 * g);
    ad = *(const float *)(unit + kActScales);
  }
};

typedef _Float16 v4h_t __attribute__((ext_vector_type(4)));
typedef float v4f_t __attribute__((ext_vector_type(4)));

// q4k_terms_v for the prefill units (a decoded with kHalfMin): imin = sum_j mn_j (lo_j + 64 hi_j) from one
// v_mfma_f32_16x16x16_f16, whose products and partial sums are integers below 2^24 (|imin| <= 8 * 63 * 4064), so
// exact in f32: the same float the integer path converts.
__device__ __forceinline__ void q4k_terms_p(const Q4kA &a, const ActBP &b, float t[4]) {
  v4i_t dlo = {0, 0, 0, 0}, dhi = {0, 0, 0, 0};
#pragma unroll
  for (int c = 0; c < 4; c++) {
    dlo = __builtin_amdgcn_mfma_i32_16x16x64_i8(a.lo[c], b.q[c], dlo, 0, 0, 0);
    dhi = __builtin_amdgcn_mfma_i32_16x16x64_i8(a.hi[c], b.q[c], dhi, 0, 0, 0);
  }
  const v4f_t mf = __builtin_amdgcn_mfma_f32_16x16x16f16(__builtin_bit_cast(v4h_t, a.mn), __builtin_bit_cast(v4h_t, b.bm),
                                                         v4f_t{0.0f, 0.0f, 0.0f, 0.0f}, 0, 0, 0);
#pragma unroll
  for (int i = 0; i < 4; i++) {
    const int isum = 8 * dhi[i] + dlo[i];
    const float dd = __fmul_rn(a.d[i], b.ad), dm = __fmul_rn(a.dmin[i], b.ad);
    const float pm = __fmul_rn(dm, mf[i]);
    t[i] = __builtin_fmaf(dd, (float)isum, -pm);
  }
}

}  // namespace c0ven
