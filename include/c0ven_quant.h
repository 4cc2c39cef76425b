/* The weight formats the MoE block reads, numbered as ggml numbers them, and their field tables.
 *
 * Replaces the reference's shared/quant.h (ids :9-33, values per block :36-44, bytes per block :47-75, field tables
 * :78-166, run offsets :172-176, QUANT_FILE_PAD :180, codebook buffer offsets :189-196). The numeric values, the field
 * order (quants first, the f16 scales last) and the codebook buffer offsets are the same, so a caller that built
 * buffers for the reference's headers builds the same bytes for these. Only the ten types this block implements on
 * the GPU (Q8_0, Q4_K, Q5_K, Q6_K, IQ3_S, IQ4_NL, IQ4_XS, Q2_0, IQ3_XXS, IQ2_S) and the two activation types (q8_0,
 * q8_K) carry field tables; the other ids are kept so that a caller's switch over them still compiles. C and HIP device code both include this header. */
#ifndef C0VEN_QUANT_H
#define C0VEN_QUANT_H

#include <stdint.h>

#if defined(__HIPCC__)
#define C0VEN_FN static inline __host__ __device__
#elif defined(__cplusplus)
#define C0VEN_FN static inline constexpr
#else
#define C0VEN_FN static inline
#endif

/* ggml type ids at llama.cpp 3cf03257 (ggml/include/ggml.h). */
#define QT_F32 0
#define QT_F16 1
#define QT_Q4_0 2
#define QT_Q5_0 6
#define QT_Q5_1 7
#define QT_Q8_0 8
#define QT_Q8_1 9
#define QT_Q2_K 10
#define QT_Q3_K 11
#define QT_Q4_K 12
#define QT_Q5_K 13
#define QT_Q6_K 14
#define QT_Q8_K 15
#define QT_IQ2_XXS 16
#define QT_IQ2_XS 17
#define QT_IQ3_XXS 18
#define QT_IQ1_S 19
#define QT_IQ4_NL 20
#define QT_IQ3_S 21
#define QT_IQ2_S 22
#define QT_IQ4_XS 23
#define QT_IQ1_M 29
#define QT_BF16 30
#define QT_Q2_0 42

#define QK_K 256 /* values per super-block */

/* Values per block. */
C0VEN_FN uint32_t quant_block_values(uint32_t t) {
  switch (t) {
    case QT_Q4_0: case QT_Q5_0: case QT_Q5_1: case QT_Q8_0: case QT_Q8_1: case QT_IQ4_NL: return 32;
    case QT_Q2_0: return 64;
    case QT_Q2_K: case QT_Q3_K: case QT_Q4_K: case QT_Q5_K: case QT_Q6_K: case QT_Q8_K:
    case QT_IQ1_S: case QT_IQ1_M: case QT_IQ2_XXS: case QT_IQ2_XS:
    case QT_IQ3_XXS: case QT_IQ3_S: case QT_IQ2_S: case QT_IQ4_XS: return 256;
    default: return 1;
  }
}

/* Bytes per block; 0 for a type no reader here knows. */
C0VEN_FN uint32_t quant_block_bytes(uint32_t t) {
  switch (t) {
    case QT_F32: return 4;
    case QT_F16: case QT_BF16: return 2;
    case QT_Q4_0: return 18;
    case QT_Q5_0: return 22;
    case QT_Q5_1: return 24;
    case QT_Q8_0: return 34;
    case QT_Q8_1: return 36;
    case QT_Q2_K: return 84;
    case QT_Q3_K: return 110;
    case QT_Q4_K: return 144;
    case QT_Q5_K: return 176;
    case QT_Q6_K: return 210;
    case QT_Q8_K: return 292;
    case QT_IQ1_S: return 50;
    case QT_IQ1_M: return 56;
    case QT_IQ2_XXS: return 66;
    case QT_IQ2_XS: return 74;
    case QT_IQ3_XXS: return 98;
    case QT_IQ4_NL: return 18;
    case QT_IQ3_S: return 110;
    case QT_IQ2_S: return 82;
    case QT_IQ4_XS: return 136;
    case QT_Q2_0: return 18;
    default: return 0;
  }
}

/* Whether the GPU block implements a weight type. */
C0VEN_FN int quant_gpu_supported(uint32_t t) {
  return t == QT_Q8_0 || t == QT_Q4_K || t == QT_Q5_K || t == QT_Q6_K || t == QT_IQ3_S || t == QT_IQ4_NL ||
         t == QT_IQ4_XS || t == QT_Q2_0 || t == QT_IQ3_XXS || t == QT_IQ2_S;
}

/* Whether a weight type decodes through a codebook the caller supplies (ggml-common.h's iq3xxs_grid and iq2s_grid,
 * which this build does not carry: moe_set_codebooks). */
C0VEN_FN int quant_needs_codebook(uint32_t t) { return t == QT_IQ3_XXS || t == QT_IQ2_S; }

/* The activation type a weight type's integer dot product takes on the CPU (ggml-cpu.c vec_dot_type): q8_K for the
 * K- and i-quants of 256-value blocks, q8_0 for Q8_0, IQ4_NL and Q2_0 (ggml-cpu.c :272, :380, :234). 0 (F32) for a
 * type without one here. */
C0VEN_FN uint32_t quant_vec_dot_type(uint32_t t) {
  switch (t) {
    case QT_Q8_0: case QT_IQ4_NL: case QT_Q2_0: return QT_Q8_0;
    case QT_Q4_K: case QT_Q5_K: case QT_Q6_K: case QT_IQ3_S: case QT_IQ4_XS: case QT_IQ3_XXS: case QT_IQ2_S:
      return QT_Q8_K;
    default: return QT_F32;
  }
}

/* Fields of a block in run order: (offset in the file's block << 8) | size. Quants first, f16 scales last. */
C0VEN_FN uint32_t quant_nfields(uint32_t t) {
  switch (t) {
    case QT_IQ3_S: case QT_IQ2_S: return 5;
    case QT_Q5_K: case QT_Q6_K: case QT_IQ4_XS: return 4;
    case QT_Q4_K: case QT_IQ3_XXS: return 3;
    case QT_Q8_0: case QT_IQ4_NL: case QT_Q2_0: return 2;
    case QT_Q8_K: return 3;
    default: return 1;
  }
}

C0VEN_FN uint32_t quant_field_(uint32_t t, uint32_t f) {
  switch (t) {
    case QT_IQ3_S: /* qs, signs, qh, scales, d */
      return f == 0 ? (2u << 8) | 64 : f == 1 ? (74u << 8) | 32 : f == 2 ? (66u << 8) | 8 : f == 3 ? (106u << 8) | 4
                                                                                                : (0u << 8) | 2;
    case QT_IQ2_S: /* qs (grid index low bits), signs, qh, scales, d */
      return f == 0 ? (2u << 8) | 32 : f == 1 ? (34u << 8) | 32 : f == 2 ? (66u << 8) | 8 : f == 3 ? (74u << 8) | 8
                                                                                                : (0u << 8) | 2;
    case QT_IQ3_XXS: /* grid indices, scale-and-sign words, d */
      return f == 0 ? (2u << 8) | 64 : f == 1 ? (66u << 8) | 32 : (0u << 8) | 2;
    case QT_Q5_K: /* qs, qh, scales, d and dmin */
      return f == 0 ? (48u << 8) | 128 : f == 1 ? (16u << 8) | 32 : f == 2 ? (4u << 8) | 12 : (0u << 8) | 4;
    case QT_Q6_K: /* ql, qh, scales, d (the file already has the f16 scale last) */
      return f == 0 ? (0u << 8) | 128 : f == 1 ? (128u << 8) | 64 : f == 2 ? (192u << 8) | 16 : (208u << 8) | 2;
    case QT_IQ4_XS: /* qs, scales_l, scales_h, d */
      return f == 0 ? (8u << 8) | 128 : f == 1 ? (4u << 8) | 4 : f == 2 ? (2u << 8) | 2 : (0u << 8) | 2;
    case QT_Q4_K: /* qs, scales, d and dmin */
      return f == 0 ? (16u << 8) | 128 : f == 1 ? (4u << 8) | 12 : (0u << 8) | 4;
    case QT_Q8_0: /* qs, d */
      return f == 0 ? (2u << 8) | 32 : (0u << 8) | 2;
    case QT_IQ4_NL: case QT_Q2_0: /* qs, d */
      return f == 0 ? (2u << 8) | 16 : (0u << 8) | 2;
    case QT_Q8_K: /* qs (256 int8), bsums (16 int16), d (f32) */
      return f == 0 ? (4u << 8) | 256 : f == 1 ? (260u << 8) | 32 : (0u << 8) | 4;
    default: return quant_block_bytes(t);
  }
}

C0VEN_FN uint32_t quant_field_offset(uint32_t t, uint32_t f) { return quant_field_(t, f) >> 8; }
C0VEN_FN uint32_t quant_field_size(uint32_t t, uint32_t f) { return quant_field_(t, f) & 0xff; }

/* Where field f's run starts in a slice of n blocks laid out as runs (one run per field, largest first). */
C0VEN_FN uint64_t quant_run_offset(uint32_t t, uint32_t f, uint64_t n) {
  uint64_t off = 0;
  for (uint32_t g = 0; g < f; g++) off += quant_field_size(t, g);
  return off * n;
}

/* Bytes a reader may touch past a slice's last block in the file's layout. */
#define QUANT_FILE_PAD 8

/* The codebook buffer's layout, as the reference packs ggml-common.h's tables for its cards (core/load/codebooks.cpp).
 * This build carries the IQ3_S grid (512 x u32) and kvalues (kvalues_iq4nl: -127 .. 113) itself; iq2s_grid and
 * iq3xxs_grid come from the caller in a buffer of this layout (moe_set_codebooks). */
#define QGRID_IQ2S 0        /* u64 x 1024 */
#define QGRID_IQ3XXS 8192   /* u32 x 256 */
#define QGRID_IQ3S 9216     /* u32 x 512 */
#define QGRID_KVALUES 11264 /* i8 x 16 (kvalues_iq4nl) */
#define QGRID_IQ2XXS 11280  /* u64 x 256 */
#define QGRID_IQ2XS 13328   /* u64 x 512 */
#define QGRID_IQ1S 17424    /* u64 x 2048 */
#define QGRID_BYTES 33808

#endif
