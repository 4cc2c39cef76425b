// The device layout of the expert matrices and of the quantised activations, shared by the host repacker and the
// kernels.
//
// A matrix of R rows x K values is a sequence of row tiles of 64 rows. A row's K values are U = K / 256 units (a
// super-block of Q4_K or IQ3_S, eight blocks of Q8_0). Inside a tile the 64 U (row, unit) pairs are numbered
// unit-major, idx = unit * 64 + row (pair_idx), and each field of the format is stored idx-minor: piece p of pair idx
// at field_base + (p * 64 U + idx) * piece_bytes, field_base being the earlier fields' bytes times 64 U. A wave's load
// of piece p then reads whole runs: the matrix-core paths' 16 or 32 rows of one unit are 256 or 512 consecutive
// bytes, the dot4 paths' eight rows of each unit (a row's units on consecutive lanes) a 128-byte line per unit. A
// work item's rows of the U units lie 64 pieces apart, spread over more memory channels than one run would be.
// The bytes are those of the file's blocks, permuted (nothing is decoded or re-rounded): the reference's runs layout
// (shared/quant.h:1-4, core/load/runs.cpp:12-31) shaped for 64-wide wavefronts.
//
//   Q8_0  (8 blocks, 272 B): qs 16 pieces x 16 B (values 16p..16p+15), then d 1 x 16 B (8 f16, block order).
//   IQ4_NL (8 blocks, 144 B): qs 8 x 16 B (block p's 16 bytes), then d 1 x 16 B (8 f16).
//   Q2_0  (4 blocks of 64, 72 B): qs 4 x 16 B (block p's 16 bytes), then d 1 x 8 B (4 f16).
//   Q4_K  (144 B):           qs 8 x 16 B (the block's qs bytes 16p..16p+15), scales 3 x 4 B, then d|dmin 1 x 4 B.
//   IQ3_S (110 B):           qs 4 x 16 B, signs 2 x 16 B, qh 2 x 4 B, scales 1 x 4 B, then d 1 x 2 B.
//   IQ3_XXS (98 B):          qs 4 x 16 B (grid indices, sub-blocks 2p, 2p+1), scale-and-sign words 2 x 16 B, d 1 x 2 B.
//   IQ2_S (82 B):            qs 2 x 16 B (index low bits, sub-blocks 4p..4p+3), signs 2 x 16 B, qh 1 x 8 B,
//                            scales 1 x 8 B, then d 1 x 2 B.
//   IQ4_XS (136 B):          qs 8 x 16 B (sub-block p's 16 bytes), then the block's first 8 bytes 1 x 8 B (d,
//                            scales_h, scales_l as the file has them).
//   Q5_K (176 B):            qs 8 x 16 B (as Q4_K), qh 2 x 16 B, scales 3 x 4 B, then d|dmin 1 x 4 B.
//   Q6_K (210 B):            ql 8 x 16 B, qh 4 x 16 B, scales 1 x 16 B, then d 1 x 2 B.
#pragma once

#include <stdint.h>

#include "../../include/c0ven_quant.h"

#if defined(__HIPCC__)
#define C0VEN_HD __host__ __device__ inline
#else
#define C0VEN_HD inline
#endif

namespace c0ven {

constexpr uint32_t kUnit = 256;     // values per unit
constexpr uint32_t kTileRows = 64;  // rows per tile

// Units of a K-value row: a partial last unit (K not a multiple of 256; types with 32-value blocks) is stored as a whole
// one whose missing blocks are zero (zero weights, zero scales).
C0VEN_HD uint32_t units_of(uint32_t k) { return (k + kUnit - 1) / kUnit; }
// The lanes the decode kernel's dot4 items give a row: the units rounded up to a power of two (lanes past the real
// units add exact zeros).
C0VEN_HD uint32_t unit_lanes(uint32_t U) {
  uint32_t l = 1;
  while (l < U) l <<= 1;
  return l;
}

C0VEN_HD uint32_t unit_bytes(uint32_t type) {
  return type == QT_Q8_0    ? 272u
         : type == QT_Q4_K  ? 144u
         : type == QT_IQ3_S ? 110u
         : type == QT_IQ4_NL ? 144u
         : type == QT_Q2_0  ? 72u
         : type == QT_IQ3_XXS ? 98u
         : type == QT_IQ2_S ? 82u
         : type == QT_IQ4_XS ? 136u
         : type == QT_Q5_K  ? 176u
         : type == QT_Q6_K  ? 210u
                            : 0u;
}
// The 256-value types whose values come from a grid codebook (decoded with the grid in LDS).
C0VEN_HD constexpr bool grid_family(uint32_t type) {
  return type == QT_IQ3_S || type == QT_IQ3_XXS || type == QT_IQ2_S;
}
// The q8_K types decoded without a codebook: their A operands come from the unit's own bytes.
C0VEN_HD constexpr bool kq_family(uint32_t type) {
  return type == QT_Q4_K || type == QT_Q5_K || type == QT_Q6_K || type == QT_IQ4_XS;
}
// The 256-value types the prefill GEMM takes block by block (one MFMA a 32-value block or half block, then the
// block's integer scale): the grid types and IQ4_XS, Q5_K, Q6_K.
C0VEN_HD constexpr bool block_scaled(uint32_t type) {
  return grid_family(type) || type == QT_IQ4_XS || type == QT_Q5_K || type == QT_Q6_K;
}
// The 32-value block types that meet q8_0 activations (one fp32 term a 32-value block, or half a Q2_0 block).
C0VEN_HD constexpr bool q8_family(uint32_t type) { return type == QT_Q8_0 || type == QT_IQ4_NL || type == QT_Q2_0; }
// The number of pair (row in tile, unit) inside its tile.
C0VEN_HD uint32_t pair_idx(uint32_t row, uint32_t u) { return u * kTileRows + row; }
// A tile of 64 rows x U units.
C0VEN_HD uint64_t tile_bytes(uint32_t type, uint32_t U) { return (uint64_t)kTileRows * U * unit_bytes(type); }

// Field bases inside a tile, in units of nl = 64 U pairs.
namespace q8_0t { constexpr uint32_t kQs = 0, kD = 16 * 16; }
namespace q4_kt { constexpr uint32_t kQs = 0, kScales = 8 * 16, kDm = 8 * 16 + 3 * 4; }
namespace iq4_nlt { constexpr uint32_t kQs = 0, kD = 8 * 16; }
namespace q2_0t { constexpr uint32_t kQs = 0, kD = 4 * 16; }
namespace iq3_xxst { constexpr uint32_t kQs = 0, kSs = 4 * 16, kD = 6 * 16; }
namespace iq2_st { constexpr uint32_t kQs = 0, kSigns = 2 * 16, kQh = 4 * 16, kScales = 4 * 16 + 8, kD = 4 * 16 + 16; }
namespace iq4_xst { constexpr uint32_t kQs = 0, kMeta = 8 * 16; }
namespace q5_kt { constexpr uint32_t kQs = 0, kQh = 8 * 16, kScales = 8 * 16 + 2 * 16, kDm = 8 * 16 + 2 * 16 + 3 * 4; }
namespace q6_kt { constexpr uint32_t kQl = 0, kQh = 8 * 16, kScales = 8 * 16 + 4 * 16, kD = 8 * 16 + 4 * 16 + 16; }
namespace iq3_st {
constexpr uint32_t kQs = 0, kSigns = 4 * 16, kQh = 6 * 16, kScales = 6 * 16 + 2 * 4, kD = 6 * 16 + 3 * 4;
}

// Bytes of an R x K matrix in the device layout (R rounded up to whole tiles).
C0VEN_HD uint64_t matrix_bytes(uint32_t type, uint32_t rows, uint32_t k) {
  const uint64_t rt = (rows + kTileRows - 1) / kTileRows;
  return rt * tile_bytes(type, units_of(k));
}

// A quantised activation unit (one token's or one assignment's 256 values), 320 B in global memory:
//   [0, 256)   the int8 codes;
//   [256, 288) the scales as f32: q8_K's d at 256; q8_0's eight block d (their f16 values widened) at 256 + 4 b;
//   [288, 320) q8_K only: the sums of each 32 codes as int32 (bsums[2j] + bsums[2j + 1]), or, in units written by
//              the prefill quantiser, the same sums split for the Q4_K minimum MFMA (kActSplitH).
// In LDS the kernels keep them kActLds apart, so the eight units a wave reads at once fall in distinct banks.
constexpr uint32_t kActBytes = 320, kActScales = 256, kActSums = 288, kActLds = 336;
// In LDS the 16 bytes of padding after a unit may hold its sums split for the Q4_K minimum MFMA (hi bytes, lo bytes).
constexpr uint32_t kActSplit = 320;
// In a q8_K unit in global memory written by the prefill quantiser, bytes 288-319 hold each block sum s_j split as
// 64 hi_j + lo_j (hi in [-64, 63], lo in [0, 63]) as f16 values: lo_0 .. lo_7, then 64 hi_0 .. 64 hi_7 (all exact in
// f16), the B operand of one v_mfma_f32_16x16x16_f16 per position tile, so that a unit can be copied to LDS verbatim.
constexpr uint32_t kActSplitH = 288;

}  // namespace c0ven
