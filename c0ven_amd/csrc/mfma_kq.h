// IQ4_XS, Q5_K and Q6_K weights against activation units on the matrix cores, in the block-scaled form of
// mfma_iq3s.h: one v_mfma_i32_16x16x32_i8 per 32-value block (two for Q6_K, whose 16-value halves have scales of their
// own) on the signed codes, each D multiplied by its integer block scale and added to the unit's int32 sum in block
// order, then the unit's fp32 term as UnitIQ4_XS / UnitQ5_K / UnitQ6_K::term (units.h) forms it.
//
// Operand layout (one wave), as in mfma_q4k.h: lane l holds A row l % 16 and B column l % 16, the values 8 g .. 8 g + 7
// of each 32-value block, g = l / 16; D[row][col] sits in lane 16 (row / 4) + col as element row % 4, so a lane needs
// the scales of D rows 4 g + i (loaded for those rows directly).
//
// Exactness: the codes are exact signed bytes (IQ4_XS kvalues -127..113, Q5_K 0..31, Q6_K -32..31); each block's D is
// the exact int32 dot, its scale (IQ4_XS ls - 32, Q5_K 0..63, Q6_K -128..127) multiplies it as an integer, and a
// unit's sum stays within int32 (at most 256 x 127 x 128 x 63 < 2^31).
#pragma once

#include "device_math.h"
#include "layout.h"
#include "units.h"

namespace c0ven {

// IQ4_XS: the lane's eight values of block ib are nibble half g / 2 of bytes 8 (g % 2) .. + 7 of sub-block ib's 16
// qs bytes (low nibbles are values 0-15, high ones 16-31).
struct Iq4xsRaw {
  uint32_t qs[16];      // block ib: words 2 ib, 2 ib + 1
  uint32_t meta[4][2];  // D row 4 g + i: (d | scales_h << 16, scales_l)
  uint32_t dh[4];
  static constexpr uint32_t kHalves = 1;
  static constexpr bool kMin = false;
  static constexpr float kFactor = 1.0f;
  __device__ __forceinline__ void load(const uint8_t *mat, uint32_t U, uint32_t row0, uint32_t u, uint32_t lane) {
    const uint32_t g = lane / 16, nl = kTileRows * U;
    const uint8_t *tile = mat + (uint64_t)(row0 / kTileRows) * tile_bytes(QT_IQ4_XS, U);
    const uint32_t ia = pair_idx((row0 % kTileRows) + lane % 16, u);
#pragma unroll
    for (uint32_t ib = 0; ib < 8; ib++) {
      const uint2 v = *(const uint2 *)(tile + ((uint64_t)ib * nl + ia) * 16 + 8 * (g % 2));
      qs[2 * ib] = v.x, qs[2 * ib + 1] = v.y;
    }
#pragma unroll
    for (uint32_t i = 0; i < 4; i++) {
      const uint32_t id = pair_idx((row0 % kTileRows) + 4 * g + i, u);
      const uint2 m = *(const uint2 *)(tile + (uint64_t)iq4_xst::kMeta * nl + (uint64_t)id * 8);
      meta[i][0] = m.x, meta[i][1] = m.y, dh[i] = m.x & 0xffffu;
    }
  }
  __device__ __forceinline__ void prep(uint32_t) {}
  __device__ __forceinline__ long a_block(uint32_t ib, uint32_t lane, const uint32_t *) const {
    const uint32_t sh = 4 * ((lane / 16) / 2);
    const uint32_t w0 = iq4nl_lookup((qs[2 * ib] >> sh) & 0x0f0f0f0fu);
    const uint32_t w1 = iq4nl_lookup((qs[2 * ib + 1] >> sh) & 0x0f0f0f0fu);
    return (long)(((uint64_t)w1 << 32) | w0);
  }
  __device__ __forceinline__ int ls(uint32_t i, uint32_t ib) const {
    return (int)(((meta[i][1] >> (4 * ib)) & 15u) | (((meta[i][0] >> (16 + 2 * ib)) & 3u) << 4)) - 32;
  }
};

// Q5_K: block ib is sub-block ib (chunk c = ib / 2 of the qs bytes, nibble ib % 2); the lane's eight values are
// bytes 32 c + 8 g .. + 7 of qs with bit ib of qh bytes 8 g .. + 7 as their fifth bit. The minimum part
// sum_j m_j bsum_j is formed from the activation units' block sums (kMin).
struct Q5kRaw {
  uint32_t qs[4][2], qh[2];
  uint32_t sc[4][3], dm[4];  // D row 4 g + i: the 12 scale bytes and d | dmin << 16
  uint32_t dh[4];
  static constexpr uint32_t kHalves = 1;
  static constexpr bool kMin = true;
  static constexpr float kFactor = 1.0f;
  __device__ __forceinline__ void load(const uint8_t *mat, uint32_t U, uint32_t row0, uint32_t u, uint32_t lane) {
    const uint32_t g = lane / 16, nl = kTileRows * U;
    const uint8_t *tile = mat + (uint64_t)(row0 / kTileRows) * tile_bytes(QT_Q5_K, U);
    const uint32_t ia = pair_idx((row0 % kTileRows) + lane % 16, u);
#pragma unroll
    for (uint32_t c = 0; c < 4; c++) {  // qs bytes 32 c + 8 g: piece 2 c + g / 2, at 8 (g % 2)
      const uint2 v = *(const uint2 *)(tile + (uint64_t)q5_kt::kQs * nl + ((uint64_t)(2 * c + g / 2) * nl + ia) * 16 +
                                       8 * (g % 2));
      qs[c][0] = v.x, qs[c][1] = v.y;
    }
    const uint2 h = *(const uint2 *)(tile + (uint64_t)q5_kt::kQh * nl + ((uint64_t)(g / 2) * nl + ia) * 16 + 8 * (g % 2));
    qh[0] = h.x, qh[1] = h.y;
#pragma unroll
    for (uint32_t i = 0; i < 4; i++) {
      const uint32_t id = pair_idx((row0 % kTileRows) + 4 * g + i, u);
#pragma unroll
      for (uint32_t k = 0; k < 3; k++)
        sc[i][k] = *(const uint32_t *)(tile + (uint64_t)q5_kt::kScales * nl + ((uint64_t)k * nl + id) * 4);
      dm[i] = *(const uint32_t *)(tile + (uint64_t)q5_kt::kDm * nl + (uint64_t)id * 4);
      dh[i] = dm[i] & 0xffffu;
    }
  }
  __device__ __forceinline__ void prep(uint32_t) {}
  __device__ __forceinline__ long a_block(uint32_t ib, uint32_t, const uint32_t *) const {
    const uint32_t c = ib / 2, sh = 4 * (ib % 2);
    const uint32_t w0 = ((qs[c][0] >> sh) & 0x0f0f0f0fu) | (((qh[0] >> ib) & 0x01010101u) << 4);
    const uint32_t w1 = ((qs[c][1] >> sh) & 0x0f0f0f0fu) | (((qh[1] >> ib) & 0x01010101u) << 4);
    return (long)(((uint64_t)w1 << 32) | w0);
  }
  // get_scale_min_k4 of sub-block j for D row 4 g + i: the scale (min = false) or the minimum.
  __device__ __forceinline__ int k4(uint32_t i, uint32_t j, bool min) const {
    const auto byte = [&](uint32_t b) { return (sc[i][b / 4] >> (8 * (b % 4))) & 0xffu; };
    if (j < 4) return (int)(byte(j + (min ? 4 : 0)) & 63u);
    return min ? (int)((byte(j + 4) >> 4) | ((byte(j) >> 6) << 4)) : (int)((byte(j + 4) & 15u) | ((byte(j - 4) >> 6) << 4));
  }
  __device__ __forceinline__ int ls(uint32_t i, uint32_t ib) const { return k4(i, ib, false); }
  __device__ __forceinline__ int mn(uint32_t i, uint32_t j) const { return k4(i, j, true); }
  __device__ __forceinline__ float dmin(uint32_t i) const { return h2f((uint16_t)(dm[i] >> 16)); }
};

// Q6_K: block ib covers values 32 ib .. (h = ib / 4, j = ib % 4); the lane's eight values l = 8 g .. + 7 take nibble
// j / 2 of ql bytes 64 h + 32 (j % 2) + l and bits 2 j of qh bytes 32 h + l, less 32. Values 0-15 and 16-31 of a
// block have scales of their own: two MFMAs a block, lanes g = 0, 1 then g = 2, 3 (as Iq2sRaw).
struct Q6kRaw {
  uint32_t ql[4][2], qh[2][2];  // ql: (h, j % 2); qh: h
  uint32_t sc[4][4];            // D row 4 g + i: its 16 scale bytes
  uint32_t dh[4];
  static constexpr uint32_t kHalves = 2;
  static constexpr bool kMin = false;
  static constexpr float kFactor = 1.0f;
  __device__ __forceinline__ void load(const uint8_t *mat, uint32_t U, uint32_t row0, uint32_t u, uint32_t lane) {
    const uint32_t g = lane / 16, nl = kTileRows * U;
    const uint8_t *tile = mat + (uint64_t)(row0 / kTileRows) * tile_bytes(QT_Q6_K, U);
    const uint32_t ia = pair_idx((row0 % kTileRows) + lane % 16, u);
#pragma unroll
    for (uint32_t s = 0; s < 4; s++) {  // ql bytes 32 s + 8 g: piece 2 s + g / 2, at 8 (g % 2)
      const uint2 v = *(const uint2 *)(tile + (uint64_t)q6_kt::kQl * nl + ((uint64_t)(2 * s + g / 2) * nl + ia) * 16 +
                                       8 * (g % 2));
      ql[s][0] = v.x, ql[s][1] = v.y;
    }
#pragma unroll
    for (uint32_t h = 0; h < 2; h++) {  // qh bytes 32 h + 8 g: piece 2 h + g / 2
      const uint2 v = *(const uint2 *)(tile + (uint64_t)q6_kt::kQh * nl + ((uint64_t)(2 * h + g / 2) * nl + ia) * 16 +
                                       8 * (g % 2));
      qh[h][0] = v.x, qh[h][1] = v.y;
    }
#pragma unroll
    for (uint32_t i = 0; i < 4; i++) {
      const uint32_t id = pair_idx((row0 % kTileRows) + 4 * g + i, u);
      const uint4 v = *(const uint4 *)(tile + (uint64_t)q6_kt::kScales * nl + (uint64_t)id * 16);
      sc[i][0] = v.x, sc[i][1] = v.y, sc[i][2] = v.z, sc[i][3] = v.w;
      dh[i] = *(const uint16_t *)(tile + (uint64_t)q6_kt::kD * nl + (uint64_t)id * 2);
    }
  }
  __device__ __forceinline__ void prep(uint32_t) {}
  __device__ __forceinline__ long a_block(uint32_t ib, uint32_t, const uint32_t *) const {
    const uint32_t h = ib / 4, j = ib % 4, s = 2 * h + j % 2, nsh = 4 * (j / 2);
    uint32_t w[2];
#pragma unroll
    for (uint32_t k = 0; k < 2; k++)
      w[k] = sub32_bytes(((ql[s][k] >> nsh) & 0x0f0f0f0fu) | (((qh[h][k] >> (2 * j)) & 0x03030303u) << 4));
    return (long)(((uint64_t)w[1] << 32) | w[0]);
  }
  // Half hh (values 16 hh ..) of block ib's scale for D row 4 g + i: scales[2 ib + hh], signed.
  __device__ __forceinline__ int ls(uint32_t i, uint32_t ib, uint32_t hh) const {
    const uint32_t b = 2 * ib + hh;
    return (int)(int8_t)((sc[i][b / 4] >> (8 * (b % 4))) & 0xffu);
  }
};

}  // namespace c0ven
