// IQ3_S weights against activation units on the matrix cores: 16 weight rows x 16 position columns x one 32-value
// block per v_mfma_i32_16x16x32_i8, with the integers and fp32 steps of UnitIQ3_S::term (units.h).
//
// Operand layout (one wave), as in mfma_q4k.h: lane l holds A row l % 16 and B column l % 16, bytes 8 g .. 8 g + 7
// of each 32-value block, g = l / 16; D[row][col] sits in lane 16 (row / 4) + col as element row % 4. A lane's eight
// bytes of block ib are the grid groups 8 ib + 2 g and 8 ib + 2 g + 1, decoded to signed bytes from the grid in LDS.
//
// Exactness: each block's D is the exact int32 dot of the signed codes with the activation codes; the block's odd
// scale ls = 1 + 2 s (at most 31, so it does not fit a folded int8 code) multiplies D as an integer and the eight
// products are added in block order, which is the CPU path's bsum.
#pragma once

#include "device_math.h"
#include "layout.h"
#include "units.h"

namespace c0ven {

// One lane's raw bytes of a 16-row x 1-unit IQ3_S tile: for its A row, the word of each block's index bytes that
// holds groups 2 g and 2 g + 1 (in halfword g % 2), the eight sign words and the two high-bit words; for its four D
// rows (4 g + i), the scales word and d.
struct Iq3sRaw {
  uint32_t qs[8], sg[8], qh[2], sc[4], dh[4];
  // Rows row0 .. row0 + 15 (row0 a multiple of 16) of the matrix at mat (U units a row), unit u.
  __device__ __forceinline__ void load(const uint8_t *mat, uint32_t U, uint32_t row0, uint32_t u, uint32_t lane) {
    const uint32_t g = lane / 16, nl = kTileRows * U;
    const uint8_t *tile = mat + (uint64_t)(row0 / kTileRows) * tile_bytes(QT_IQ3_S, U);
    const uint32_t ia = pair_idx((row0 % kTileRows) + lane % 16, u);
#pragma unroll
    for (uint32_t ib = 0; ib < 8; ib++)  // qs piece ib / 2 holds blocks 2 p (bytes 0-7) and 2 p + 1 (bytes 8-15)
      qs[ib] = *(const uint32_t *)(tile + ((uint64_t)(ib / 2) * nl + ia) * 16 + 8 * (ib % 2) + 4 * (g / 2));
#pragma unroll
    for (uint32_t p = 0; p < 2; p++) {
      const uint4 v = *(const uint4 *)(tile + (uint64_t)iq3_st::kSigns * nl + ((uint64_t)p * nl + ia) * 16);
      sg[4 * p] = v.x, sg[4 * p + 1] = v.y, sg[4 * p + 2] = v.z, sg[4 * p + 3] = v.w;
    }
#pragma unroll
    for (uint32_t p = 0; p < 2; p++)
      qh[p] = *(const uint32_t *)(tile + (uint64_t)iq3_st::kQh * nl + ((uint64_t)p * nl + ia) * 4);
#pragma unroll
    for (uint32_t i = 0; i < 4; i++) {
      const uint32_t id = pair_idx((row0 % kTileRows) + 4 * g + i, u);
      sc[i] = *(const uint32_t *)(tile + (uint64_t)iq3_st::kScales * nl + (uint64_t)id * 4);
      dh[i] = *(const uint16_t *)(tile + (uint64_t)iq3_st::kD * nl + (uint64_t)id * 2);
    }
  }
  // The A operand of block ib: groups k = 8 ib + 2 g + j (j = 0, 1), each four signed bytes (grid bytes, negated
  // where the group's sign bits are set), as UnitIQ3_S::load decodes them.
  __device__ __forceinline__ long a_block(uint32_t ib, uint32_t lane, const uint32_t *grid) const {
    const uint32_t g = lane / 16;
    uint32_t w[2];
#pragma unroll
    for (uint32_t j = 0; j < 2; j++) {
      const uint32_t byte = (qs[ib] >> (8 * (2 * (g % 2) + j))) & 0xffu;
      const uint32_t hb = (qh[ib / 4] >> (8 * (ib % 4) + 2 * g + j)) & 1u;
      const uint32_t gv = grid[byte | (hb << 8)];
      const uint32_t nib = (sg[ib] >> (4 * (2 * g + j))) & 15u;
      const uint32_t x = (nib * 0x00204081u) & 0x01010101u;  // byte t = bit t of the nibble
      w[j] = (gv ^ ((x << 8) - x)) + x;                      // grid bytes >= 1: negation has no carries
    }
    return (long)(((uint64_t)w[1] << 32) | w[0]);
  }
  // Block ib's scale of D row 4 g + i: 1 + 2 s.
  __device__ __forceinline__ int ls(uint32_t i, uint32_t ib) const { return 1 + 2 * (int)((sc[i] >> (4 * ib)) & 15u); }
  __device__ __forceinline__ void prep(uint32_t) {}
  static constexpr float kFactor = 1.0f;  // the super-block term: kFactor ((d d_a) isum)
  static constexpr uint32_t kHalves = 1;  // MFMAs a block (2: its 16-value halves have scales of their own)
  static constexpr bool kMin = false;     // a minimum term from the activations' block sums (Q5_K)
};

// IQ3_XXS (UnitIQ3_XXS::term): the lane's eight bytes of block ib are its groups 2 g and 2 g + 1, the block's sign
// group g of the A row's scale-and-sign word, the eighth sign the parity of the seven. The scales of the D rows come
// from the lanes holding those rows as A rows (one packed word each, four shuffles a unit).
struct Iq3xxsRaw {
  uint32_t qs[8], ss[8], sc[4], dh[4];
  __device__ __forceinline__ void load(const uint8_t *mat, uint32_t U, uint32_t row0, uint32_t u, uint32_t lane) {
    const uint32_t g = lane / 16, nl = kTileRows * U;
    const uint8_t *tile = mat + (uint64_t)(row0 / kTileRows) * tile_bytes(QT_IQ3_XXS, U);
    const uint32_t ia = pair_idx((row0 % kTileRows) + lane % 16, u);
#pragma unroll
    for (uint32_t ib = 0; ib < 8; ib++)  // qs piece ib / 2 holds blocks 2 p (bytes 0-7) and 2 p + 1 (bytes 8-15)
      qs[ib] = *(const uint32_t *)(tile + ((uint64_t)(ib / 2) * nl + ia) * 16 + 8 * (ib % 2) + 4 * (g / 2));
#pragma unroll
    for (uint32_t p = 0; p < 2; p++) {
      const uint4 v = *(const uint4 *)(tile + (uint64_t)iq3_xxst::kSs * nl + ((uint64_t)p * nl + ia) * 16);
      ss[4 * p] = v.x, ss[4 * p + 1] = v.y, ss[4 * p + 2] = v.z, ss[4 * p + 3] = v.w;
    }
#pragma unroll
    for (uint32_t i = 0; i < 4; i++) {
      const uint32_t id = pair_idx((row0 % kTileRows) + 4 * g + i, u);
      dh[i] = *(const uint16_t *)(tile + (uint64_t)iq3_xxst::kD * nl + (uint64_t)id * 2);
    }
  }
  // The D rows' scale nibbles (row 4 g + i: block ib at bits 4 ib of sc[i]), from their A-row lanes.
  __device__ __forceinline__ void prep(uint32_t lane) {
    uint32_t mine = 0;
#pragma unroll
    for (uint32_t ib = 0; ib < 8; ib++) mine |= (ss[ib] >> 28) << (4 * ib);
#pragma unroll
    for (uint32_t i = 0; i < 4; i++) sc[i] = (uint32_t)__shfl((int)mine, (int)(4 * (lane / 16) + i), 64);
  }
  __device__ __forceinline__ long a_block(uint32_t ib, uint32_t lane, const uint32_t *grid) const {
    const uint32_t g = lane / 16;
    const uint32_t s7 = (ss[ib] >> (7 * g)) & 127u, sb = s7 | ((uint32_t)(__popc(s7) & 1) << 7);
    uint32_t w[2];
#pragma unroll
    for (uint32_t j = 0; j < 2; j++)
      w[j] = sign4(grid[(qs[ib] >> (8 * (2 * (g % 2) + j))) & 0xffu], (sb >> (4 * j)) & 15u);
    return (long)(((uint64_t)w[1] << 32) | w[0]);
  }
  __device__ __forceinline__ int ls(uint32_t i, uint32_t ib) const { return 1 + 2 * (int)((sc[i] >> (4 * ib)) & 15u); }
  static constexpr float kFactor = 0.25f;
  static constexpr uint32_t kHalves = 1;
  static constexpr bool kMin = false;
};

// IQ2_S (UnitIQ2_S::term): the lane's eight bytes of block ib are group g of it (a 10-bit grid index into iq2s_grid,
// two words an entry, and a sign byte). Values 0-15 and 16-31 of a block have scales of their own, so each block is
// two MFMAs, one with lanes g = 0, 1 of A and one with lanes g = 2, 3 (the others zero); the D rows' scale bytes come
// from their A-row lanes.
struct Iq2sRaw {
  uint32_t qs[8], sg[8], qh[2], scw[2], sc[4][2], dh[4];
  static constexpr uint32_t kHalves = 2;
  static constexpr bool kMin = false;
  __device__ __forceinline__ void load(const uint8_t *mat, uint32_t U, uint32_t row0, uint32_t u, uint32_t lane) {
    const uint32_t g = lane / 16, nl = kTileRows * U;
    const uint8_t *tile = mat + (uint64_t)(row0 / kTileRows) * tile_bytes(QT_IQ2_S, U);
    const uint32_t ia = pair_idx((row0 % kTileRows) + lane % 16, u);
#pragma unroll
    for (uint32_t p = 0; p < 2; p++) {
      const uint4 v = *(const uint4 *)(tile + (uint64_t)iq2_st::kQs * nl + ((uint64_t)p * nl + ia) * 16);
      const uint4 t = *(const uint4 *)(tile + (uint64_t)iq2_st::kSigns * nl + ((uint64_t)p * nl + ia) * 16);
      qs[4 * p] = v.x, qs[4 * p + 1] = v.y, qs[4 * p + 2] = v.z, qs[4 * p + 3] = v.w;
      sg[4 * p] = t.x, sg[4 * p + 1] = t.y, sg[4 * p + 2] = t.z, sg[4 * p + 3] = t.w;
    }
    const uint2 h = *(const uint2 *)(tile + (uint64_t)iq2_st::kQh * nl + (uint64_t)ia * 8);
    const uint2 c = *(const uint2 *)(tile + (uint64_t)iq2_st::kScales * nl + (uint64_t)ia * 8);
    qh[0] = h.x, qh[1] = h.y, scw[0] = c.x, scw[1] = c.y;
    (void)g;
#pragma unroll
    for (uint32_t i = 0; i < 4; i++) {
      const uint32_t id = pair_idx((row0 % kTileRows) + 4 * (lane / 16) + i, u);
      dh[i] = *(const uint16_t *)(tile + (uint64_t)iq2_st::kD * nl + (uint64_t)id * 2);
    }
  }
  __device__ __forceinline__ void prep(uint32_t lane) {
#pragma unroll
    for (uint32_t i = 0; i < 4; i++)
#pragma unroll
      for (uint32_t k = 0; k < 2; k++) sc[i][k] = (uint32_t)__shfl((int)scw[k], (int)(4 * (lane / 16) + i), 64);
  }
  // Block ib's A operand: group g (values 8 g .. 8 g + 7) of its four, all lanes (a_half masks it).
  __device__ __forceinline__ long a_block(uint32_t ib, uint32_t lane, const uint32_t *grid) const {
    const uint32_t g = lane / 16, gi = 4 * ib + g;
    const uint32_t ix = ((qs[gi / 4] >> (8 * (gi % 4))) & 0xffu) | (((qh[ib / 4] >> (8 * (ib % 4) + 2 * g)) & 3u) << 8);
    const uint32_t sb = (sg[gi / 4] >> (8 * (gi % 4))) & 0xffu;
    const uint32_t w0 = sign4(grid[2 * ix], sb & 15u), w1 = sign4(grid[2 * ix + 1], sb >> 4);
    return (long)(((uint64_t)w1 << 32) | w0);
  }
  // Half h (values 16 h .. 16 h + 15) of block ib's scale for D row 4 g + i: 1 + 2 s.
  __device__ __forceinline__ int ls(uint32_t i, uint32_t ib, uint32_t h) const {
    return 1 + 2 * (int)((sc[i][ib / 4] >> (8 * (ib % 4) + 4 * h)) & 15u);
  }
  static constexpr float kFactor = 0.125f;
};

}  // namespace c0ven
