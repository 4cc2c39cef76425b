// The host's repack of a matrix from the file's layout (ggml blocks, row-major) into the device layout (layout.h).
#pragma once

#include <cstring>
#include <vector>

#include "layout.h"

namespace c0ven {

// Row r's unit u in the file's layout: the bytes of its blocks (Q8_0: 8 blocks of 34 B; IQ4_NL: 8 of 18 B; Q2_0: 4
// of 18 B; the 256-value types: one block).
inline const uint8_t *file_unit(const uint8_t *m, uint32_t type, uint32_t k, uint32_t r, uint32_t u) {
  const uint64_t row = (uint64_t)k / quant_block_values(type) * quant_block_bytes(type);
  return m + r * row + (uint64_t)u * unit_bytes(type);
}

// One unit's bytes into pair idx of a tile of nl = 64 U pairs.
inline void put_unit(uint8_t *tile, uint32_t type, uint32_t idx, uint32_t nl, const uint8_t *b) {
  auto at = [&](uint32_t base, uint32_t p, uint32_t piece) { return tile + (uint64_t)base * nl + ((uint64_t)p * nl + idx) * piece; };
  switch (type) {
    case QT_Q8_0:
      for (uint32_t p = 0; p < 16; p++) std::memcpy(at(q8_0t::kQs, p, 16), b + (p / 2) * 34 + 2 + (p % 2) * 16, 16);
      for (uint32_t blk = 0; blk < 8; blk++) std::memcpy(at(q8_0t::kD, 0, 16) + 2 * blk, b + blk * 34, 2);
      break;
    case QT_Q4_K:
      for (uint32_t p = 0; p < 8; p++) std::memcpy(at(q4_kt::kQs, p, 16), b + 16 + 16 * p, 16);
      for (uint32_t i = 0; i < 3; i++) std::memcpy(at(q4_kt::kScales, i, 4), b + 4 + 4 * i, 4);
      std::memcpy(at(q4_kt::kDm, 0, 4), b, 4);
      break;
    case QT_IQ4_NL:
      for (uint32_t p = 0; p < 8; p++) std::memcpy(at(iq4_nlt::kQs, p, 16), b + 18 * p + 2, 16);
      for (uint32_t blk = 0; blk < 8; blk++) std::memcpy(at(iq4_nlt::kD, 0, 16) + 2 * blk, b + 18 * blk, 2);
      break;
    case QT_Q2_0:
      for (uint32_t p = 0; p < 4; p++) std::memcpy(at(q2_0t::kQs, p, 16), b + 18 * p + 2, 16);
      for (uint32_t blk = 0; blk < 4; blk++) std::memcpy(at(q2_0t::kD, 0, 8) + 2 * blk, b + 18 * blk, 2);
      break;
    case QT_IQ3_XXS:
      for (uint32_t p = 0; p < 4; p++) std::memcpy(at(iq3_xxst::kQs, p, 16), b + 2 + 16 * p, 16);
      for (uint32_t p = 0; p < 2; p++) std::memcpy(at(iq3_xxst::kSs, p, 16), b + 66 + 16 * p, 16);
      std::memcpy(at(iq3_xxst::kD, 0, 2), b, 2);
      break;
    case QT_IQ2_S:
      for (uint32_t p = 0; p < 2; p++) std::memcpy(at(iq2_st::kQs, p, 16), b + 2 + 16 * p, 16);
      for (uint32_t p = 0; p < 2; p++) std::memcpy(at(iq2_st::kSigns, p, 16), b + 34 + 16 * p, 16);
      std::memcpy(at(iq2_st::kQh, 0, 8), b + 66, 8);
      std::memcpy(at(iq2_st::kScales, 0, 8), b + 74, 8);
      std::memcpy(at(iq2_st::kD, 0, 2), b, 2);
      break;
    case QT_IQ4_XS:
      for (uint32_t p = 0; p < 8; p++) std::memcpy(at(iq4_xst::kQs, p, 16), b + 8 + 16 * p, 16);
      std::memcpy(at(iq4_xst::kMeta, 0, 8), b, 8);
      break;
    case QT_Q5_K:
      for (uint32_t p = 0; p < 8; p++) std::memcpy(at(q5_kt::kQs, p, 16), b + 48 + 16 * p, 16);
      for (uint32_t p = 0; p < 2; p++) std::memcpy(at(q5_kt::kQh, p, 16), b + 16 + 16 * p, 16);
      for (uint32_t i = 0; i < 3; i++) std::memcpy(at(q5_kt::kScales, i, 4), b + 4 + 4 * i, 4);
      std::memcpy(at(q5_kt::kDm, 0, 4), b, 4);
      break;
    case QT_Q6_K:
      for (uint32_t p = 0; p < 8; p++) std::memcpy(at(q6_kt::kQl, p, 16), b + 16 * p, 16);
      for (uint32_t p = 0; p < 4; p++) std::memcpy(at(q6_kt::kQh, p, 16), b + 128 + 16 * p, 16);
      std::memcpy(at(q6_kt::kScales, 0, 16), b + 192, 16);
      std::memcpy(at(q6_kt::kD, 0, 2), b + 208, 2);
      break;
    case QT_IQ3_S:
      for (uint32_t p = 0; p < 4; p++) std::memcpy(at(iq3_st::kQs, p, 16), b + 2 + 16 * p, 16);
      for (uint32_t p = 0; p < 2; p++) std::memcpy(at(iq3_st::kSigns, p, 16), b + 74 + 16 * p, 16);
      for (uint32_t i = 0; i < 2; i++) std::memcpy(at(iq3_st::kQh, i, 4), b + 66 + 4 * i, 4);
      std::memcpy(at(iq3_st::kScales, 0, 4), b + 106, 4);
      std::memcpy(at(iq3_st::kD, 0, 2), b, 2);
      break;
  }
}

// rows x k values of type: file layout -> device layout (dst has matrix_bytes(type, rows, k); rows past the last of
// the final tile are zero, which decodes to zero weights). A partial last unit (k % 256, 32-value block types) takes
// its blocks and leaves the rest zero.
inline void repack_matrix(uint32_t type, const uint8_t *src, uint32_t rows, uint32_t k, uint8_t *dst) {
  const uint32_t U = units_of(k), nrt = (rows + kTileRows - 1) / kTileRows, nl = kTileRows * U;
  const uint64_t tb = tile_bytes(type, U);
  const uint32_t bv = quant_block_values(type), bb = quant_block_bytes(type);
  std::vector<uint8_t> part(unit_bytes(type));
  std::memset(dst, 0, matrix_bytes(type, rows, k));
  for (uint32_t rt = 0; rt < nrt; rt++) {
    uint8_t *tile = dst + (uint64_t)rt * tb;
    for (uint32_t l = 0; l < kTileRows && rt * kTileRows + l < rows; l++)
      for (uint32_t u = 0; u < U; u++) {
        const uint8_t *b = file_unit(src, type, k, rt * kTileRows + l, u);
        if ((u + 1) * kUnit > k) {  // the partial last unit: its blocks, then zero blocks
          std::memset(part.data(), 0, part.size());
          std::memcpy(part.data(), b, (uint64_t)(k - u * kUnit) / bv * bb);
          b = part.data();
        }
        put_unit(tile, type, pair_idx(l, u), nl, b);
      }
  }
}

}  // namespace c0ven
