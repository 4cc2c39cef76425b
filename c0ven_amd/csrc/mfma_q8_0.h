// Q8_0 weights against q8_0 activation units on the matrix cores: 16 weight rows x 16 position columns x one 32-value
// block per v_mfma_i32_16x16x32_i8 (the exact int32 block dot), with the fp32 steps of UnitQ8_0::term (units.h): each
// block's term (d_w d_a) dot, the eight terms of a unit added as a pairwise tree.
//
// Operand layout (one wave), as in mfma_q4k.h: lane l holds A row l % 16 and B column l % 16, bytes 8 g .. 8 g + 7
// of each block, g = l / 16; D[row][col] sits in lane 16 (row / 4) + col as element row % 4.
#pragma once

#include "device_math.h"
#include "layout.h"
#include "units.h"

namespace c0ven {

// One lane's raw bytes of a 16-row x 1-unit Q8_0 tile: its A row's eight bytes of each block, and the eight f16 block
// scales of each of its four D rows (4 g + i).
struct Q80Raw {
  long qs[8];
  uint4 dv[4];
  // Rows row0 .. row0 + 15 (row0 a multiple of 16) of the matrix at mat (U units a row), unit u.
  __device__ __forceinline__ void load(const uint8_t *mat, uint32_t U, uint32_t row0, uint32_t u, uint32_t lane) {
    const uint32_t g = lane / 16, nl = kTileRows * U;
    const uint8_t *tile = mat + (uint64_t)(row0 / kTileRows) * tile_bytes(QT_Q8_0, U);
    const uint32_t ia = pair_idx((row0 % kTileRows) + lane % 16, u);
#pragma unroll
    for (uint32_t j = 0; j < 8; j++)  // block j is qs pieces 2 j (values 0-15) and 2 j + 1 (16-31)
      qs[j] = *(const long *)(tile + ((uint64_t)(2 * j + g / 2) * nl + ia) * 16 + 8 * (g % 2));
#pragma unroll
    for (uint32_t i = 0; i < 4; i++) {
      const uint32_t id = pair_idx((row0 % kTileRows) + 4 * g + i, u);
      dv[i] = *(const uint4 *)(tile + (uint64_t)q8_0t::kD * nl + (uint64_t)id * 16);
    }
  }
  __device__ __forceinline__ void widen(uint32_t) {}  // the codes are the bytes
  // Block j's scale of D row 4 g + i.
  __device__ __forceinline__ float d(uint32_t i, uint32_t j) const {
    const uint32_t w[4] = {dv[i].x, dv[i].y, dv[i].z, dv[i].w};
    return h2f((uint16_t)(w[j / 2] >> (16 * (j % 2))));
  }
};

// The same operands for IQ4_NL (the lane's eight codes of block j looked up in kvalues_iq4nl) and Q2_0 (half j of block
// j / 2 as codes q - 1, its scale the block's): the Q8_0 kernel's steps then apply unchanged.
struct Iq4nlRaw {
  long qs[8];
  uint4 dv[4];
  __device__ __forceinline__ void load(const uint8_t *mat, uint32_t U, uint32_t row0, uint32_t u, uint32_t lane) {
    const uint32_t g = lane / 16, nl = kTileRows * U;
    const uint8_t *tile = mat + (uint64_t)(row0 / kTileRows) * tile_bytes(QT_IQ4_NL, U);
    const uint32_t ia = pair_idx((row0 % kTileRows) + lane % 16, u);
#pragma unroll
    for (uint32_t j = 0; j < 8; j++) {  // values 8 g .. 8 g + 7: nibbles (g / 2 high) of bytes 8 (g % 2) .. + 7
      const uint2 b = *(const uint2 *)(tile + ((uint64_t)(iq4_nlt::kQs / 16 + j) * nl + ia) * 16 + 8 * (g % 2));
      qs[j] = (long)(((uint64_t)b.y << 32) | b.x);  // raw bytes: widen() looks the nibbles up
    }
#pragma unroll
    for (uint32_t i = 0; i < 4; i++) {
      const uint32_t id = pair_idx((row0 % kTileRows) + 4 * g + i, u);
      dv[i] = *(const uint4 *)(tile + (uint64_t)iq4_nlt::kD * nl + (uint64_t)id * 16);
    }
  }
  // The codes from the raw bytes load left in qs (done once they have arrived, so that a load of the next unit
  // holds only the raw words).
  __device__ __forceinline__ void widen(uint32_t lane) {
    const uint32_t sh = 4 * (lane / 32);
#pragma unroll
    for (uint32_t j = 0; j < 8; j++) {
      const uint64_t b = (uint64_t)qs[j];
      qs[j] = (long)(((uint64_t)iq4nl_lookup(((uint32_t)(b >> 32) >> sh) & 0x0f0f0f0fu) << 32) |
                     iq4nl_lookup(((uint32_t)b >> sh) & 0x0f0f0f0fu));
    }
  }
  __device__ __forceinline__ float d(uint32_t i, uint32_t j) const {
    const uint32_t w[4] = {dv[i].x, dv[i].y, dv[i].z, dv[i].w};
    return h2f((uint16_t)(w[j / 2] >> (16 * (j % 2))));
  }
};

struct Q20Raw {
  long qs[8];
  uint2 dv[4];
  __device__ __forceinline__ void load(const uint8_t *mat, uint32_t U, uint32_t row0, uint32_t u, uint32_t lane) {
    const uint32_t g = lane / 16, nl = kTileRows * U;
    const uint8_t *tile = mat + (uint64_t)(row0 / kTileRows) * tile_bytes(QT_Q2_0, U);
    const uint32_t ia = pair_idx((row0 % kTileRows) + lane % 16, u);
#pragma unroll
    for (uint32_t j = 0; j < 8; j++) {  // half j: values 8 g .. 8 g + 7 are bytes 8 (j % 2) + 2 g, + 1 of block j / 2
      qs[j] = *(const uint16_t *)(tile + ((uint64_t)(q2_0t::kQs / 16 + j / 2) * nl + ia) * 16 + 8 * (j % 2) + 2 * g);
    }  // raw bytes: widen() spreads the codes
#pragma unroll
    for (uint32_t i = 0; i < 4; i++) {
      const uint32_t id = pair_idx((row0 % kTileRows) + 4 * g + i, u);
      dv[i] = *(const uint2 *)(tile + (uint64_t)q2_0t::kD * nl + (uint64_t)id * 8);
    }
  }
  __device__ __forceinline__ void widen(uint32_t) {
#pragma unroll
    for (uint32_t j = 0; j < 8; j++) {
      const uint32_t b = (uint32_t)qs[j];
      qs[j] = (long)(((uint64_t)q2_spread(b >> 8) << 32) | q2_spread(b & 0xffu));
    }
  }
  __device__ __forceinline__ float d(uint32_t i, uint32_t j) const {
    const uint32_t w = (j / 4) ? dv[i].y : dv[i].x;
    return h2f((uint16_t)(w >> (16 * ((j / 2) % 2))));
  }
};

}  // namespace c0ven
