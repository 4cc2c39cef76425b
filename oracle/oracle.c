/* TEST INFRASTRUCTURE - the CPU oracle of the MoE block (see oracle.h). Built by oracle/Makefile with
 * -ffp-contract=off, so every fp32 step rounds where the source says it does. */
#include "oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

#include "iq3s_lattice.h"

#define QT_Q8_0 8
#define QT_Q4_K 12
#define QT_Q8_K 15
#define QT_IQ3_S 21
#define QT_IQ4_NL 20
#define QT_Q2_0 42
#define QT_IQ3_XXS 18
#define QT_IQ2_S 22
#define QT_Q5_K 13
#define QT_Q6_K 14
#define QT_IQ4_XS 23
#define QGRID_IQ2S 0
#define QGRID_IQ3XXS 8192
#define QK 256

/* kvalues_iq4nl (ggml-common.h:1120-1122): the IQ4_NL codebook, which must hash to QUANT_FORMATS.md:547's sha256
 * (tests/test_oracle.py checks it). */
static const int8_t kIq4nl[16] = {-127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113};

void orc_iq4nl_values(int8_t *out) { memcpy(out, kIq4nl, 16); }

/* ---------------------------------------------------------------------------------------------------------------
 * Scalars. */

/* IEEE binary16 from binary32, rounded to nearest even (what F16C's vcvtps2ph with mode 0 and ggml's
 * GGML_FP32_TO_FP16 give). */
uint16_t orc_fp32_to_fp16(float f) {
  uint32_t x;
  memcpy(&x, &f, 4);
  const uint32_t sign = (x >> 16) & 0x8000u, ax = x & 0x7fffffffu;
  if (ax >= 0x7f800000u) return (uint16_t)(sign | (ax > 0x7f800000u ? 0x7e00u : 0x7c00u));
  if (ax >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u); /* 65520 and up round to infinity */
  if (ax < 0x38800000u) {                                   /* below 2^-14: a subnormal half, units of 2^-24 */
    float a;
    memcpy(&a, &ax, 4);
    return (uint16_t)(sign | (uint32_t)nearbyintf(a * 16777216.0f));
  }
  uint32_t h = ((((ax >> 23) - 112u) << 10) | ((ax & 0x7fffffu) >> 13));
  const uint32_t rem = ax & 0x1fffu;
  if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h++;
  return (uint16_t)(sign | h);
}

float orc_fp16_to_fp32(uint16_t h) {
  const uint32_t sign = (uint32_t)(h & 0x8000u) << 16, e = (h >> 10) & 31u, m = h & 0x3ffu;
  uint32_t x;
  if (e == 0) {
    float v = (float)m * (1.0f / 16777216.0f); /* exact: m < 2^10 */
    memcpy(&x, &v, 4);
    x |= sign;
  } else if (e == 31) {
    x = sign | 0x7f800000u | (m << 13);
  } else {
    x = sign | ((e + 112u) << 23) | (m << 13);
  }
  float f;
  memcpy(&f, &x, 4);
  return f;
}

/* bf16 by round to nearest even, NaN kept quiet (ggml-impl.h GGML_FP32_TO_BF16). */
uint16_t orc_fp32_to_bf16(float f) {
  uint32_t x;
  memcpy(&x, &f, 4);
  if ((x & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((x >> 16) | 64u);
  return (uint16_t)((x + (0x7fffu + ((x >> 16) & 1u))) >> 16);
}

static inline float bf16_to_fp32(uint16_t b) {
  const uint32_t x = (uint32_t)b << 16;
  float f;
  memcpy(&f, &x, 4);
  return f;
}

void orc_expf(const float *x, float *y, int64_t n) {
  for (int64_t i = 0; i < n; i++) y[i] = expf(x[i]);
}

/* ggml's nearest_int (ggml-quants.c): round half to even through the float adder, for |v| < 2^22. */
static inline int nearest_int(float v) {
  const float t = v + 12582912.0f;
  int32_t i;
  memcpy(&i, &t, 4);
  return (i & 0x007fffff) - 0x00400000;
}

/* ---------------------------------------------------------------------------------------------------------------
 * The IQ3_S codebook: entry i is four bytes 2 l_j + 1 (j = 0..3, byte j), l_j the 3-bit fields of the lattice code
 * kIq3sLattice[i] (l_0 in bits 0-2). These are the 512 points ggml's iq3xs_init_impl(512) (ggml-quants.c) builds
 * iq3s_grid from; their table must hash to QUANT_FORMATS.md:546's sha256, which tests/test_oracle.py checks. */
static uint32_t g_grid[512];
static int g_grid_ready;

static void grid_init(void) {
  if (g_grid_ready) return;
  for (int i = 0; i < 512; i++) {
    const uint32_t c = kIq3sLattice[i];
    uint32_t v = 0;
    for (int j = 0; j < 4; j++) v |= (2u * ((c >> (3 * j)) & 7u) + 1u) << (8 * j);
    g_grid[i] = v;
  }
  g_grid_ready = 1;
}

void orc_iq3s_grid(uint32_t *out) {
  grid_init();
  memcpy(out, g_grid, sizeof g_grid);
}

/* ---------------------------------------------------------------------------------------------------------------
 * Decoders (ggml-quants.c dequantize_row_*, as QUANT_FORMATS.md states them). */

static inline uint16_t rd16(const uint8_t *p) { return (uint16_t)(p[0] | (p[1] << 8)); }

/* Q4_K's packed 6-bit scale and minimum of sub-block j (get_scale_min_k4, QUANT_FORMATS.md:383-389). */
static inline void scale_min_k4(int j, const uint8_t *q, int *sc, int *m) {
  if (j < 4) {
    *sc = q[j] & 63;
    *m = q[j + 4] & 63;
  } else {
    *sc = (q[j + 4] & 0xF) | ((q[j - 4] >> 6) << 4);
    *m = (q[j + 4] >> 4) | ((q[j] >> 6) << 4);
  }
}

/* iq2s_grid and iq3xxs_grid, which ggml-common.h holds and this repository does not: the caller's, from a buffer in
 * the QGRID layout (core/load/codebooks.cpp:14-33 packs ggml's tables so). */
static uint64_t g_iq2s[1024];
static uint32_t g_iq3xxs[256];

void orc_set_codebooks(const uint8_t *qgrid) {
  memcpy(g_iq2s, qgrid + QGRID_IQ2S, sizeof g_iq2s);
  memcpy(g_iq3xxs, qgrid + QGRID_IQ3XXS, sizeof g_iq3xxs);
}

/* Value v of an IQ3_XXS block (QUANT_FORMATS.md:147-166): (grid magnitude, negative?) and the sub-block's scale
 * nibble s. Sign group l = (v % 32) / 8 of sub-block b is the 7-bit index (w >> 7 l) & 127 of the sub-block's word,
 * its eighth bit the index's parity (ksigns_iq2xs). */
static inline void iq3xxs_value(const uint8_t *b, int v, int *mag, int *neg, int *s) {
  const int ib = v / 32, j = v % 32, l = j / 8;
  uint32_t w;
  memcpy(&w, b + 66 + 4 * ib, 4);
  const uint32_t idx7 = (w >> (7 * l)) & 127u, sb = idx7 | ((uint32_t)(__builtin_popcount(idx7) & 1) << 7);
  const uint8_t q = b[2 + 8 * ib + 2 * l + (j % 8) / 4];
  *mag = (int)((g_iq3xxs[q] >> (8 * (j % 4))) & 0xffu);
  *neg = (int)((sb >> (j % 8)) & 1u);
  *s = (int)(w >> 28);
}

/* Value v of an IQ2_S block (QUANT_FORMATS.md:115-137): (grid magnitude, negative?) and its half sub-block's scale
 * nibble (low nibble for values 0-15 of the sub-block, high for 16-31). */
static inline void iq2s_value(const uint8_t *b, int v, int *mag, int *neg, int *s) {
  const int ib = v / 32, j = v % 32, g = j / 8;
  const uint32_t idx = b[2 + 4 * ib + g] | (((uint32_t)(b[66 + ib] >> (2 * g)) & 3u) << 8);
  *mag = (int)((g_iq2s[idx] >> (8 * (j % 8))) & 0xffu);
  *neg = (int)((b[34 + 4 * ib + g] >> (j % 8)) & 1u);
  *s = (int)((b[74 + ib] >> (4 * (j / 16))) & 15u);
}

/* Value v of an IQ3_S block as (grid magnitude, negative?) with its sub-block scale 1 + 2 s. */
static inline void iq3s_value(const uint8_t *b, int v, int *mag, int *neg, int *ls) {
  const uint8_t *qs = b + 2, *qh = b + 66, *signs = b + 74, *scales = b + 106;
  const int ib = v / 32, k = (v % 32) / 4, j = v % 4, l = (v % 32) / 8;
  const uint32_t idx = qs[8 * ib + k] | (((qh[ib] >> k) & 1u) << 8);
  *mag = (int)((g_grid[idx] >> (8 * j)) & 0xffu);
  *neg = (signs[4 * ib + l] >> (v % 8)) & 1;
  *ls = 1 + 2 * ((scales[ib / 2] >> (4 * (ib % 2))) & 15);
}

/* Q5_K value v's code 0..31: the Q4_K nibble (chunk v / 64: byte v % 32 of it, high nibble for the second 32) and
 * bit v / 32 of qh byte v % 32 as bit 4 (QUANT_FORMATS.md:405-411). */
static inline int q5k_code(const uint8_t *b, int v) {
  const uint8_t *qs = b + 48, *qh = b + 16;
  const int c = v / 64, l = v % 32, hi = (v % 64) / 32;
  const int q4 = hi ? qs[32 * c + l] >> 4 : qs[32 * c + l] & 15;
  return q4 | (((qh[l] >> (v / 32)) & 1) << 4);
}

/* Q6_K value v's code less 32, by the table of QUANT_FORMATS.md:433-441: h = v / 128, j = (v % 128) / 32, l = v % 32;
 * the low four bits are nibble j / 2 of ql[64 h + 32 (j % 2) + l], the high two bits 2 j of qh[32 h + l]. */
static inline int q6k_code(const uint8_t *b, int v) {
  const int h = v / 128, j = (v % 128) / 32, l = v % 32;
  const int lo = (b[64 * h + 32 * (j % 2) + l] >> (4 * (j / 2))) & 15;
  const int hi = (b[128 + 32 * h + l] >> (2 * j)) & 3;
  return (lo | (hi << 4)) - 32;
}

/* IQ4_XS sub-block ib's scale less 32: bits 0-3 from scales_l byte ib / 2 (low nibble for even ib), bits 4-5 from
 * bits 2 ib of scales_h (QUANT_FORMATS.md:217-224). */
static inline int iq4xs_scale(const uint8_t *b, int ib) {
  const int lo = (b[4 + ib / 2] >> (4 * (ib % 2))) & 15, hi = (rd16(b + 2) >> (2 * ib)) & 3;
  return (lo | (hi << 4)) - 32;
}
/* IQ4_XS value v's nibble: byte 16 (v / 32) + v % 16 of qs, low nibble for v % 32 < 16. */
static inline int iq4xs_nibble(const uint8_t *b, int v) {
  const uint8_t q = b[8 + 16 * (v / 32) + v % 16];
  return (v % 32) < 16 ? q & 15 : q >> 4;
}

int orc_dequantize_row(uint32_t type, const void *src, float *dst, int64_t n) {
  const uint8_t *b = (const uint8_t *)src;
  grid_init();
  switch (type) {
    case QT_Q8_0: /* y = d q (quants.c:553-567) */
      if (n % 32) return -1;
      for (int64_t i = 0; i < n / 32; i++, b += 34) {
        const float d = orc_fp16_to_fp32(rd16(b));
        for (int j = 0; j < 32; j++) dst[32 * i + j] = d * (float)(int8_t)b[2 + j];
      }
      return 0;
    case QT_Q4_K: /* y = (d sc) q - (dmin m) (quants.c:1529-1551) */
      if (n % QK) return -1;
      for (int64_t i = 0; i < n / QK; i++, b += 144) {
        const float d = orc_fp16_to_fp32(rd16(b)), dmin = orc_fp16_to_fp32(rd16(b + 2));
        const uint8_t *q = b + 16;
        float *y = dst + QK * i;
        for (int c = 0; c < 4; c++, q += 32) {
          int sc, m;
          scale_min_k4(2 * c, b + 4, &sc, &m);
          const float d1 = d * (float)sc, m1 = dmin * (float)m;
          scale_min_k4(2 * c + 1, b + 4, &sc, &m);
          const float d2 = d * (float)sc, m2 = dmin * (float)m;
          for (int l = 0; l < 32; l++) y[64 * c + l] = d1 * (float)(q[l] & 0xF) - m1;
          for (int l = 0; l < 32; l++) y[64 * c + 32 + l] = d2 * (float)(q[l] >> 4) - m2;
        }
      }
      return 0;
    case QT_IQ3_S: /* y = (d (1 + 2 s)) grid sign (quants.c:2607-2646) */
      if (n % QK) return -1;
      for (int64_t i = 0; i < n / QK; i++, b += 110) {
        const float d = orc_fp16_to_fp32(rd16(b));
        for (int v = 0; v < QK; v++) {
          int mag, neg, ls;
          iq3s_value(b, v, &mag, &neg, &ls);
          const float db = d * (float)ls;
          dst[QK * i + v] = db * (float)mag * (neg ? -1.0f : 1.0f);
        }
      }
      return 0;
    case QT_IQ4_NL: /* y = d kvalues[nibble]; byte j holds value j (low nibble) and j + 16 (QUANT_FORMATS.md:234-245) */
      if (n % 32) return -1;
      for (int64_t i = 0; i < n / 32; i++, b += 18) {
        const float d = orc_fp16_to_fp32(rd16(b));
        for (int j = 0; j < 16; j++) {
          dst[32 * i + j] = d * (float)kIq4nl[b[2 + j] & 15];
          dst[32 * i + j + 16] = d * (float)kIq4nl[b[2 + j] >> 4];
        }
      }
      return 0;
    case QT_Q2_0: /* y = (q - 1) d, value j bits 2 (j mod 4) of byte j / 4 (QUANT_FORMATS.md:251-262, quants.c:439-457) */
      if (n % 64) return -1;
      for (int64_t i = 0; i < n / 64; i++, b += 18) {
        const float d = orc_fp16_to_fp32(rd16(b));
        for (int j = 0; j < 64; j++) dst[64 * i + j] = (float)((int)((b[2 + j / 4] >> (2 * (j % 4))) & 3) - 1) * d;
      }
      return 0;
    case QT_Q5_K: /* y = (d sc) (q4 + 16 h) - (dmin m) (QUANT_FORMATS.md:401-417, quants.c:1731-1756) */
      if (n % QK) return -1;
      for (int64_t i = 0; i < n / QK; i++, b += 176) {
        const float d = orc_fp16_to_fp32(rd16(b)), dmin = orc_fp16_to_fp32(rd16(b + 2));
        for (int v = 0; v < QK; v++) {
          int sc, m;
          scale_min_k4(v / 32, b + 4, &sc, &m);
          const float dl = d * (float)sc, ml = dmin * (float)m;
          dst[QK * i + v] = dl * (float)q5k_code(b, v) - ml;
        }
      }
      return 0;
    case QT_Q6_K: /* y = (d sc[v / 16]) (q - 32) (QUANT_FORMATS.md:419-445, quants.c:1939-1968) */
      if (n % QK) return -1;
      for (int64_t i = 0; i < n / QK; i++, b += 210) {
        const float d = orc_fp16_to_fp32(rd16(b + 208));
        for (int v = 0; v < QK; v++) dst[QK * i + v] = d * (float)(int8_t)b[192 + v / 16] * (float)q6k_code(b, v);
      }
      return 0;
    case QT_IQ4_XS: /* y = (d (ls - 32)) kvalues[nibble] (QUANT_FORMATS.md:213-232, quants.c:2743-2764) */
      if (n % QK) return -1;
      for (int64_t i = 0; i < n / QK; i++, b += 136) {
        const float d = orc_fp16_to_fp32(rd16(b));
        for (int v = 0; v < QK; v++) {
          const float dl = d * (float)iq4xs_scale(b, v / 32);
          dst[QK * i + v] = dl * (float)kIq4nl[iq4xs_nibble(b, v)];
        }
      }
      return 0;
    case QT_IQ3_XXS: /* y = ((d (0.5 + s)) 0.5) grid sign (quants.c:2575-2603) */
      if (n % QK) return -1;
      for (int64_t i = 0; i < n / QK; i++, b += 98) {
        const float d = orc_fp16_to_fp32(rd16(b));
        for (int v = 0; v < QK; v++) {
          int mag, neg, sc;
          iq3xxs_value(b, v, &mag, &neg, &sc);
          const float db = d * (0.5f + (float)sc) * 0.5f;
          dst[QK * i + v] = db * (float)mag * (neg ? -1.0f : 1.0f);
        }
      }
      return 0;
    case QT_IQ2_S: /* y = ((d (0.5 + s)) 0.25) grid sign (quants.c:2543-2571) */
      if (n % QK) return -1;
      for (int64_t i = 0; i < n / QK; i++, b += 82) {
        const float d = orc_fp16_to_fp32(rd16(b));
        for (int v = 0; v < QK; v++) {
          int mag, neg, sc;
          iq2s_value(b, v, &mag, &neg, &sc);
          const float db = d * (0.5f + (float)sc) * 0.25f;
          dst[QK * i + v] = db * (float)mag * (neg ? -1.0f : 1.0f);
        }
      }
      return 0;
    default: return -1;
  }
}

/* ---------------------------------------------------------------------------------------------------------------
 * Activation quantisers. */

/* q8_0 as ggml's x86 quantize_row_q8_0 makes it: d = amax / 127 stored as f16, codes round(x * (127 / amax)) to
 * nearest even (QUANT_FORMATS.md:463-465 gives the rule; the AVX2 kernel scales by 127/amax and rounds with
 * _MM_ROUND_NEAREST). */
static void quantize_q8_0(const float *x, uint8_t *y, int64_t n) {
  for (int64_t i = 0; i < n / 32; i++, x += 32, y += 34) {
    float amax = 0.0f;
    for (int j = 0; j < 32; j++) amax = fmaxf(amax, fabsf(x[j]));
    const float d = amax / 127.0f, id = amax != 0.0f ? 127.0f / amax : 0.0f;
    const uint16_t dh = orc_fp32_to_fp16(d);
    y[0] = (uint8_t)(dh & 0xff);
    y[1] = (uint8_t)(dh >> 8);
    for (int j = 0; j < 32; j++) y[2 + j] = (uint8_t)(int8_t)nearest_int(x[j] * id);
  }
}

/* q8_K (quantize_row_q8_K_ref, QUANT_FORMATS.md:528-535): the value of largest magnitude max, iscale = -127 / max,
 * q = min(127, nearest(iscale x)), d = 1 / iscale (f32), bsums the sums of each 16 codes. An all-zero block is d = 0,
 * codes and sums 0. Layout: d f32 at 0, qs at 4, bsums int16 at 260 (292 B). */
static void quantize_q8_K(const float *x, uint8_t *y, int64_t n) {
  for (int64_t i = 0; i < n / QK; i++, x += QK, y += 292) {
    float max = 0.0f, amax = 0.0f;
    for (int j = 0; j < QK; j++) {
      const float ax = fabsf(x[j]);
      if (ax > amax) {
        amax = ax;
        max = x[j];
      }
    }
    int8_t *qs = (int8_t *)(y + 4);
    int16_t bs[16];
    if (amax == 0.0f) {
      memset(y, 0, 292);
      continue;
    }
    const float iscale = -127.0f / max;
    for (int j = 0; j < QK; j++) {
      const int v = nearest_int(iscale * x[j]);
      qs[j] = (int8_t)(v < 127 ? v : 127);
    }
    for (int j = 0; j < 16; j++) {
      int s = 0;
      for (int l = 0; l < 16; l++) s += qs[16 * j + l];
      bs[j] = (int16_t)s;
    }
    memcpy(y + 260, bs, 32);
    const float d = 1.0f / iscale;
    memcpy(y, &d, 4);
  }
}

int orc_quantize_act(uint32_t act_type, const float *src, void *dst, int64_t n) {
  if (act_type == QT_Q8_0 && n % 32 == 0) {
    quantize_q8_0(src, (uint8_t *)dst, n);
    return 0;
  }
  if (act_type == QT_Q8_K && n % QK == 0) {
    quantize_q8_K(src, (uint8_t *)dst, n);
    return 0;
  }
  return -1;
}

/* The 32-value block types: q8_0 activations (ggml-cpu.c vec_dot_type: Q8_0, IQ4_NL :380, Q2_0 :234). */
static int q8_family(uint32_t t) { return t == QT_Q8_0 || t == QT_IQ4_NL || t == QT_Q2_0; }
static uint32_t act_type_of(uint32_t t) {
  return q8_family(t) ? QT_Q8_0
         : (t == QT_Q4_K || t == QT_Q5_K || t == QT_Q6_K || t == QT_IQ3_S || t == QT_IQ4_XS || t == QT_IQ3_XXS ||
            t == QT_IQ2_S)
             ? QT_Q8_K
             : 0;
}
static uint64_t act_bytes(uint32_t act, uint64_t n) { return act == QT_Q8_0 ? n / 32 * 34 : n / QK * 292; }
static uint64_t row_bytes(uint32_t t, uint64_t n) {
  return t == QT_Q8_0 ? n / 32 * 34
         : t == QT_IQ4_NL ? n / 32 * 18
         : t == QT_Q2_0   ? n / 64 * 18
         : t == QT_Q4_K   ? n / QK * 144
         : t == QT_IQ3_S  ? n / QK * 110
         : t == QT_IQ3_XXS ? n / QK * 98
         : t == QT_IQ2_S  ? n / QK * 82
         : t == QT_IQ4_XS ? n / QK * 136
         : t == QT_Q5_K   ? n / QK * 176
         : t == QT_Q6_K   ? n / QK * 210
                          : 0;
}
/* The values a row's length must be a multiple of: the type's block. */
static int64_t row_block(uint32_t t) { return t == QT_Q8_0 || t == QT_IQ4_NL ? 32 : t == QT_Q2_0 ? 64 : QK; }

/* ---------------------------------------------------------------------------------------------------------------
 * Block dot products. Each returns the block's fp32 term; the row sums them in ORACLE ORDER: a pairwise tree within
 * each unit of 256 values (Q8_0's eight blocks; a Q4_K or IQ3_S super-block is one term), the units in sequence. */

static float pairwise(const float *a, int64_t n) {
  if (n == 1) return a[0];
  int64_t m = 1;
  while (2 * m < n) m *= 2;
  return pairwise(a, m) + pairwise(a + m, n - m);
}

/* Q8_0 x q8_0 (vec_dot_q8_0_q8_0, QUANT_FORMATS.md:468-470): (d_w d_a) sum q_w q_a. */
static float term_q8_0(const uint8_t *w, const uint8_t *a) {
  int32_t s = 0;
  for (int j = 0; j < 32; j++) s += (int32_t)(int8_t)w[2 + j] * (int32_t)(int8_t)a[2 + j];
  const float d = orc_fp16_to_fp32(rd16(w)) * orc_fp16_to_fp32(rd16(a));
  return d * (float)s;
}

/* IQ4_NL x q8_0 (vec_dot_iq4_nl_q8_0, QUANT_FORMATS.md:243-246): (d_w d_a) sum kvalues[nibble] q_a. */
static float term_iq4_nl(const uint8_t *w, const uint8_t *a) {
  int32_t s = 0;
  for (int j = 0; j < 16; j++)
    s += kIq4nl[w[2 + j] & 15] * (int32_t)(int8_t)a[2 + j] + kIq4nl[w[2 + j] >> 4] * (int32_t)(int8_t)a[2 + j + 16];
  const float d = orc_fp16_to_fp32(rd16(w)) * orc_fp16_to_fp32(rd16(a));
  return d * (float)s;
}

/* Q2_0 x q8_0, half h (0, 1) of a 64-value block against one 32-value q8_0 block (QUANT_FORMATS.md:264-270: one
 * term a half, d d_a sumi with the codes unpacked to q - 1): (d_w d_a) sum (q - 1) q_a. */
static float term_q2_0(const uint8_t *w, int h, const uint8_t *a) {
  int32_t s = 0;
  for (int j = 0; j < 32; j++) {
    const int v = 32 * h + j;
    s += ((int)((w[2 + v / 4] >> (2 * (v % 4))) & 3) - 1) * (int32_t)(int8_t)a[2 + j];
  }
  const float d = orc_fp16_to_fp32(rd16(w)) * orc_fp16_to_fp32(rd16(a));
  return d * (float)s;
}

/* Q4_K x q8_K (vec_dot_q4_K_q8_K, QUANT_FORMATS.md:391-400): the scale part sum_j sc_j sum q q_a and the minimum part
 * sum_j m_j (bsums of sub-block j), both exact integers, then (d_w d_a) isum - (dmin_w d_a) imin with one rounding
 * for the second product and a fused multiply-add for the first. */
static float term_q4_K(const uint8_t *w, const uint8_t *a) {
  float ad;
  memcpy(&ad, a, 4);
  const int8_t *q8 = (const int8_t *)(a + 4);
  int16_t bs[16];
  memcpy(bs, a + 260, 32);
  const uint8_t *q = w + 16;
  int32_t isum = 0, imin = 0;
  for (int j = 0; j < 8; j++) {
    int sc, m;
    scale_min_k4(j, w + 4, &sc, &m);
    const uint8_t *qc = q + 32 * (j / 2);
    int32_t dot = 0;
    for (int l = 0; l < 32; l++) dot += (int32_t)((j & 1) ? qc[l] >> 4 : qc[l] & 0xF) * q8[32 * j + l];
    isum += sc * dot;
    imin += m * (bs[2 * j] + bs[2 * j + 1]);
  }
  const float d = orc_fp16_to_fp32(rd16(w)) * ad, dm = orc_fp16_to_fp32(rd16(w + 2)) * ad;
  const float pm = dm * (float)imin;
  return fmaf(d, (float)isum, -pm);
}

/* IQ3_S x q8_K (vec_dot_iq3_s_q8_K; core/cpu/multirow.cpp:179-245 states its integer steps): per sub-block
 * (1 + 2 s) sum grid sign q_a, summed as an integer, times (d_w d_a). */
static float term_iq3_s(const uint8_t *w, const uint8_t *a) {
  float ad;
  memcpy(&ad, a, 4);
  const int8_t *q8 = (const int8_t *)(a + 4);
  int32_t bsum = 0;
  for (int ib = 0; ib < 8; ib++) {
    int32_t s = 0, ls = 0;
    for (int i = 0; i < 32; i++) {
      int mag, neg;
      iq3s_value(w, 32 * ib + i, &mag, &neg, &ls);
      s += (neg ? -mag : mag) * q8[32 * ib + i];
    }
    bsum += ls * s;
  }
  const float d = orc_fp16_to_fp32(rd16(w)) * ad;
  return d * (float)bsum;
}

/* IQ3_XXS x q8_K (vec_dot_iq3_xxs_q8_K; core/cpu/multirow.cpp:126-176 states its integer steps): per sub-block
 * (2 s + 1) sum grid sign q_a, summed as an integer, then 0.25 ((d_w d_a) isum) (the power of two exact). */
static float term_iq3_xxs(const uint8_t *w, const uint8_t *a) {
  float ad;
  memcpy(&ad, a, 4);
  const int8_t *q8 = (const int8_t *)(a + 4);
  int32_t isum = 0;
  for (int ib = 0; ib < 8; ib++) {
    int32_t s = 0;
    int sc = 0;
    for (int i = 0; i < 32; i++) {
      int mag, neg;
      iq3xxs_value(w, 32 * ib + i, &mag, &neg, &sc);
      s += (neg ? -mag : mag) * q8[32 * ib + i];
    }
    isum += (2 * sc + 1) * s;
  }
  const float d = orc_fp16_to_fp32(rd16(w)) * ad;
  return 0.25f * (d * (float)isum);
}

/* IQ2_S x q8_K (vec_dot_iq2_s_q8_K; core/cpu/multirow.cpp:68-124): per half sub-block (2 s + 1) sum grid sign q_a,
 * summed as an integer, then 0.125 ((d_w d_a) isum). */
static float term_iq2_s(const uint8_t *w, const uint8_t *a) {
  float ad;
  memcpy(&ad, a, 4);
  const int8_t *q8 = (const int8_t *)(a + 4);
  int32_t isum = 0;
  for (int h = 0; h < 16; h++) {
    int32_t s = 0;
    int sc = 0;
    for (int i = 0; i < 16; i++) {
      int mag, neg;
      iq2s_value(w, 16 * h + i, &mag, &neg, &sc);
      s += (neg ? -mag : mag) * q8[16 * h + i];
    }
    isum += (2 * sc + 1) * s;
  }
  const float d = orc_fp16_to_fp32(rd16(w)) * ad;
  return 0.125f * (d * (float)isum);
}

/* Q5_K x q8_K (vec_dot_q5_K_q8_K): Q4_K's term with the five-bit codes. */
static float term_q5_K(const uint8_t *w, const uint8_t *a) {
  float ad;
  memcpy(&ad, a, 4);
  const int8_t *q8 = (const int8_t *)(a + 4);
  int16_t bs[16];
  memcpy(bs, a + 260, 32);
  int32_t isum = 0, imin = 0;
  for (int j = 0; j < 8; j++) {
    int sc, m;
    scale_min_k4(j, w + 4, &sc, &m);
    int32_t dot = 0;
    for (int l = 0; l < 32; l++) dot += q5k_code(w, 32 * j + l) * q8[32 * j + l];
    isum += sc * dot;
    imin += m * (bs[2 * j] + bs[2 * j + 1]);
  }
  const float d = orc_fp16_to_fp32(rd16(w)) * ad, dm = orc_fp16_to_fp32(rd16(w + 2)) * ad;
  const float pm = dm * (float)imin;
  return fmaf(d, (float)isum, -pm);
}

/* Q6_K x q8_K (vec_dot_q6_K_q8_K, QUANT_FORMATS.md:443-445): per sub-block of 16 its signed scale times the exact
 * dot of (q - 32) with q_a, summed as an integer, then (d_w d_a) isum. */
static float term_q6_K(const uint8_t *w, const uint8_t *a) {
  float ad;
  memcpy(&ad, a, 4);
  const int8_t *q8 = (const int8_t *)(a + 4);
  int32_t isum = 0;
  for (int s = 0; s < 16; s++) {
    int32_t dot = 0;
    for (int l = 0; l < 16; l++) dot += q6k_code(w, 16 * s + l) * q8[16 * s + l];
    isum += (int32_t)(int8_t)w[192 + s] * dot;
  }
  const float d = orc_fp16_to_fp32(rd16(w + 208)) * ad;
  return d * (float)isum;
}

/* IQ4_XS x q8_K (vec_dot_iq4_xs_q8_K, QUANT_FORMATS.md:230-232): per sub-block (ls - 32) times the exact dot of
 * kvalues[nibble] with q_a, summed as an integer, then (d_w d_a) isum. */
static float term_iq4_xs(const uint8_t *w, const uint8_t *a) {
  float ad;
  memcpy(&ad, a, 4);
  const int8_t *q8 = (const int8_t *)(a + 4);
  int32_t isum = 0;
  for (int ib = 0; ib < 8; ib++) {
    int32_t dot = 0;
    for (int l = 0; l < 32; l++) dot += kIq4nl[iq4xs_nibble(w, 32 * ib + l)] * q8[32 * ib + l];
    isum += iq4xs_scale(w, ib) * dot;
  }
  const float d = orc_fp16_to_fp32(rd16(w)) * ad;
  return d * (float)isum;
}

static float dot_row(uint32_t type, int64_t n, const uint8_t *w, const uint8_t *a, float *terms) {
  int64_t nb;
  switch (type) {
    case QT_Q8_0:
      nb = n / 32;
      for (int64_t i = 0; i < nb; i++) terms[i] = term_q8_0(w + 34 * i, a + 34 * i);
      break;
    case QT_IQ4_NL:
      nb = n / 32;
      for (int64_t i = 0; i < nb; i++) terms[i] = term_iq4_nl(w + 18 * i, a + 34 * i);
      break;
    case QT_Q2_0:  /* two terms a block, one per 32-value half */
      nb = n / 32;
      for (int64_t i = 0; i < nb; i++) terms[i] = term_q2_0(w + 18 * (i / 2), (int)(i % 2), a + 34 * i);
      break;
    case QT_Q4_K:
      nb = n / QK;
      for (int64_t i = 0; i < nb; i++) terms[i] = term_q4_K(w + 144 * i, a + 292 * i);
      break;
    case QT_IQ3_XXS:
      nb = n / QK;
      for (int64_t i = 0; i < nb; i++) terms[i] = term_iq3_xxs(w + 98 * i, a + 292 * i);
      break;
    case QT_IQ2_S:
      nb = n / QK;
      for (int64_t i = 0; i < nb; i++) terms[i] = term_iq2_s(w + 82 * i, a + 292 * i);
      break;
    case QT_Q5_K:
      nb = n / QK;
      for (int64_t i = 0; i < nb; i++) terms[i] = term_q5_K(w + 176 * i, a + 292 * i);
      break;
    case QT_Q6_K:
      nb = n / QK;
      for (int64_t i = 0; i < nb; i++) terms[i] = term_q6_K(w + 210 * i, a + 292 * i);
      break;
    case QT_IQ4_XS:
      nb = n / QK;
      for (int64_t i = 0; i < nb; i++) terms[i] = term_iq4_xs(w + 136 * i, a + 292 * i);
      break;
    default:
      nb = n / QK;
      for (int64_t i = 0; i < nb; i++) terms[i] = term_iq3_s(w + 110 * i, a + 292 * i);
      break;
  }
  const int64_t per = q8_family(type) ? 8 : 1;  /* terms a unit of 256 values has */
  float acc = 0.0f;
  for (int64_t i = 0; i < nb; i += per) acc += pairwise(terms + i, nb - i < per ? nb - i : per);
  return acc;
}

int orc_vec_dot(uint32_t type, int64_t n, const void *w_row, const void *act, float *out) {
  if (!act_type_of(type) || n % row_block(type) || n <= 0) return -1;
  grid_init();
  float *terms = (float *)malloc(sizeof(float) * (size_t)(n / 32));
  *out = dot_row(type, n, (const uint8_t *)w_row, (const uint8_t *)act, terms);
  free(terms);
  return 0;
}

/* ---------------------------------------------------------------------------------------------------------------
 * CpuExperts (core/cpu/experts.cpp). */

/* silu(g) * u with the optional clamp (experts.cpp:21-27): g / (1 + e^-g) * u, libm's expf. */
static inline float swiglu_one(float g, float u, float limit) {
  if (limit > 0.0f) {
    g = fminf(g, limit);
    u = u < -limit ? -limit : (u > limit ? limit : u);
  }
  return g / (1.0f + expf(-g)) * u;
}

static int shape_ok(const orc_shape *s) {
  const uint32_t ga = act_type_of(s->gate_type), da = act_type_of(s->down_type);
  if (!ga || !da || !s->n_embd || !s->n_ff) return 0;
  if (s->up_type && act_type_of(s->up_type) != ga) return 0;  /* gate and up read one quantised x */
  if (s->n_embd % row_block(s->gate_type) || s->n_ff % row_block(s->down_type)) return 0;
  return 1;
}

static void quantize_act_row(uint32_t act, const float *x, uint8_t *y, int64_t n) {
  if (act == QT_Q8_0)
    quantize_q8_0(x, y, n);
  else
    quantize_q8_K(x, y, n);
}

int orc_compute_many(const orc_shape *s, const orc_job *jobs, uint32_t njobs, uint32_t ntok, const float *x,
                     uint64_t x_stride, float *y, uint64_t y_stride, int nthreads) {
  const uint32_t E = s->n_embd, F = s->n_ff;
  if (njobs == 0) {
    for (uint32_t t = 0; t < ntok; t++) memset(y + t * y_stride, 0, sizeof(float) * E);
    return 0;
  }
  if (!shape_ok(s)) return -1;
  for (uint32_t j = 0; j < njobs; j++)
    if (jobs[j].tok >= ntok || !jobs[j].gate || !jobs[j].up || !jobs[j].down) return -1;
  grid_init();
  if (nthreads <= 0) nthreads = 1;
  const uint32_t ga = act_type_of(s->gate_type), da = act_type_of(s->down_type);
  const uint64_t xq_bytes = act_bytes(ga, E), hq_bytes = act_bytes(da, F);
  const uint32_t ut = s->up_type ? s->up_type : s->gate_type;
  const uint64_t grow = row_bytes(s->gate_type, E), urow = row_bytes(ut, E), drow = row_bytes(s->down_type, F);
  const uint32_t nterm = (E > F ? E : F) / 32;
  uint8_t *xq = (uint8_t *)malloc(ntok * xq_bytes);
  uint8_t *hq = (uint8_t *)malloc(njobs * hq_bytes);
  float *h = (float *)malloc(sizeof(float) * njobs * F);
  float *out = (float *)malloc(sizeof(float) * njobs * E);
  uint32_t *dj = (uint32_t *)malloc(sizeof(uint32_t) * njobs); /* jobs ordered by distinct expert */
  uint32_t *dstart = (uint32_t *)malloc(sizeof(uint32_t) * (njobs + 1));
  if (!xq || !hq || !h || !out || !dj || !dstart) {
    free(xq), free(hq), free(h), free(out), free(dj), free(dstart);
    return -1;
  }
  for (uint32_t t = 0; t < ntok; t++) quantize_act_row(ga, x + t * x_stride, xq + t * xq_bytes, E);
  /* The distinct experts by pointer equality on gate (experts.cpp:170-177), each with its jobs in order, so that an
   * expert's rows are read once for all of them. */
  uint32_t nd = 0, nj = 0;
  {
    uint8_t *taken = (uint8_t *)calloc(njobs, 1);
    for (uint32_t j = 0; j < njobs; j++) {
      if (taken[j]) continue;
      dstart[nd++] = nj;
      for (uint32_t i = j; i < njobs; i++)
        if (!taken[i] && jobs[i].gate == jobs[j].gate) taken[i] = 1, dj[nj++] = i;
    }
    dstart[nd] = nj;
    free(taken);
  }
  const int64_t tasks_gu = (int64_t)nd * F;
#pragma omp parallel num_threads(nthreads)
  {
    float terms[nterm];
#pragma omp for schedule(static)
    for (int64_t task = 0; task < tasks_gu; task++) {
      const uint32_t d = (uint32_t)(task / F), r = (uint32_t)(task % F);
      for (uint32_t i = dstart[d]; i < dstart[d + 1]; i++) {
        const orc_job *jb = &jobs[dj[i]];
        const uint8_t *xa = xq + jb->tok * xq_bytes;
        const float g = dot_row(s->gate_type, E, jb->gate + r * grow, xa, terms);
        const float u = dot_row(ut, E, jb->up + r * urow, xa, terms);
        h[(uint64_t)dj[i] * F + r] = swiglu_one(g, u, s->swiglu_limit);
      }
    }
  }
  /* h quantised whole per job: compute_many's blocks never straddle its task rows (experts.cpp:194-238), so this is
   * the same bytes. */
  for (uint32_t j = 0; j < njobs; j++) quantize_act_row(da, h + (uint64_t)j * F, hq + j * hq_bytes, F);
  const int64_t tasks_d = (int64_t)nd * E;
#pragma omp parallel num_threads(nthreads)
  {
    float terms[nterm];
#pragma omp for schedule(static)
    for (int64_t task = 0; task < tasks_d; task++) {
      const uint32_t d = (uint32_t)(task / E), r = (uint32_t)(task % E);
      for (uint32_t i = dstart[d]; i < dstart[d + 1]; i++) {
        const uint32_t j = dj[i];
        out[(uint64_t)j * E + r] = dot_row(s->down_type, F, jobs[j].down + r * drow, hq + j * hq_bytes, terms);
      }
    }
  }
  /* y overwritten, then each token's jobs added in the order given (experts.cpp:256-262): y += w out, the product
   * rounded before the sum. */
  for (uint32_t t = 0; t < ntok; t++) memset(y + t * y_stride, 0, sizeof(float) * E);
  for (uint32_t j = 0; j < njobs; j++) {
    float *yt = y + jobs[j].tok * y_stride;
    const float w = jobs[j].w;
    for (uint32_t r = 0; r < E; r++) yt[r] = yt[r] + w * out[(uint64_t)j * E + r];
  }
  free(xq), free(hq), free(h), free(out), free(dj), free(dstart);
  return 0;
}

/* CpuExperts::compute (experts.cpp:109-150): one token; the same arithmetic as compute_many with every job on it. */
int orc_compute(const orc_shape *s, const uint8_t *const *gate, const uint8_t *const *up, const uint8_t *const *down,
                const float *w, uint32_t n, const float *x, float *y) {
  orc_job *jobs = (orc_job *)malloc(sizeof(orc_job) * (n ? n : 1));
  for (uint32_t i = 0; i < n; i++) {
    jobs[i].gate = gate[i], jobs[i].up = up[i], jobs[i].down = down[i];
    jobs[i].tok = 0, jobs[i].w = w[i];
  }
  const int rc = orc_compute_many(s, jobs, n, 1, x, s->n_embd, y, s->n_embd, 1);
  free(jobs);
  return rc;
}

/* ---------------------------------------------------------------------------------------------------------------
 * The router (MODEL_LAYER.md:414-425). */

/* The logits of one token: x rounded to bf16 (MODEL_LAYER.md:512), each product of two bf16 values exact in fp32,
 * their sum taken in double and rounded once to fp32. ggml's BF16 vec_dot sums in an order of its own (unpinned);
 * this is the exactly-rounded value it approximates. The bias, when given, is added after (not in the reference:
 * the synthetic configs' Zipf skew). */
static void logits_row(const uint16_t *router, const float *bias, uint32_t E, uint32_t H, const float *x,
                       float *lg) {
  uint16_t *xb = (uint16_t *)malloc(sizeof(uint16_t) * H);
  for (uint32_t i = 0; i < H; i++) xb[i] = orc_fp32_to_bf16(x[i]);
  for (uint32_t e = 0; e <= E; e++) {
    const uint16_t *wr = router + (uint64_t)e * H;
    double acc = 0.0;
    for (uint32_t i = 0; i < H; i++) acc += (double)(bf16_to_fp32(wr[i]) * bf16_to_fp32(xb[i]));
    float v = (float)acc;
    if (bias && e < E) v = v + bias[e];
    lg[e] = v;
  }
  free(xb);
}

/* Softmax, the top k, the weights for one token (route.h:33-99, layer.cl:765-804, ggml soft_max):
 * P_e = expf(l_e - max) * (float)(1 / sum_e expf(l_e - max)), the sum in double in expert order; the k largest
 * logits (so the k largest P), larger first, ties to the lower expert, -0 equal to +0; w_k = P_k / max(sum of the
 * k P in rank order, 6.1035e-5). */
static void topk_row(const float *lg, uint32_t E, uint32_t k, int32_t *ids, float *w) {
  float mx = -INFINITY;
  for (uint32_t e = 0; e < E; e++) mx = fmaxf(mx, lg[e]);
  double sum = 0.0;
  for (uint32_t e = 0; e < E; e++) sum += (double)expf(lg[e] - mx);
  const float inv = (float)(1.0 / sum);
  uint8_t *taken = (uint8_t *)calloc(E, 1);
  float p[64];
  for (uint32_t r = 0; r < k; r++) {
    int32_t best = -1;
    for (uint32_t e = 0; e < E; e++) {
      if (taken[e]) continue;
      if (best < 0 || lg[e] > lg[best]) best = (int32_t)e; /* strictly larger: an equal one keeps the lower id */
    }
    taken[best] = 1;
    ids[r] = best;
    p[r] = expf(lg[best] - mx) * inv;
  }
  float tot = 0.0f;
  for (uint32_t r = 0; r < k; r++) tot = tot + p[r];
  const float den = fmaxf(tot, 6.1035e-5f);
  for (uint32_t r = 0; r < k; r++) w[r] = p[r] / den;
  free(taken);
}

int orc_topk_logits(const float *logits, uint32_t n_expert, uint32_t k, int32_t *ids, float *w) {
  if (!n_expert || k == 0 || k > n_expert || k > 64) return -1;
  topk_row(logits, n_expert, k, ids, w);
  return 0;
}

int orc_route(const uint16_t *router, const float *bias, uint32_t n_expert, uint32_t n_embd, uint32_t k,
              const float *x, uint32_t ntok, uint64_t x_stride, float *logits, int32_t *ids, float *w) {
  if (!router || !n_expert || !n_embd || k == 0 || k > n_expert || k > 64) return -1;
  float *lg = (float *)malloc(sizeof(float) * (n_expert + 1));
  for (uint32_t t = 0; t < ntok; t++) {
    logits_row(router, bias, n_expert, n_embd, x + t * x_stride, lg);
    if (logits) memcpy(logits + (uint64_t)t * (n_expert + 1), lg, sizeof(float) * (n_expert + 1));
    topk_row(lg, n_expert, k, ids + (uint64_t)t * k, w + (uint64_t)t * k);
  }
  free(lg);
  return 0;
}

/* ---------------------------------------------------------------------------------------------------------------
 * The block (MODEL_LAYER.md section 4): y = sum_k w_k y_k (rank order, as compute_many sums its jobs) + gs s, the
 * product gs s rounded before the sum, gs = 1 / (1 + expf(-l_E)). */
int orc_moe_forward(const orc_layer *L, const float *x, uint32_t ntok, uint64_t x_stride, float *y, uint64_t y_stride,
                    int32_t *ids_out, float *w_out, int nthreads) {
  const uint32_t E = L->n_expert, H = L->n_embd, k = L->n_used;
  if (ntok == 0) return 0;
  float *lg = (float *)malloc(sizeof(float) * ntok * (E + 1));
  int32_t *ids = (int32_t *)malloc(sizeof(int32_t) * ntok * k);
  float *w = (float *)malloc(sizeof(float) * ntok * k);
  orc_job *jobs = (orc_job *)malloc(sizeof(orc_job) * ntok * k);
  float *s = (float *)malloc(sizeof(float) * ntok * H);
  int rc = orc_route(L->router, L->bias, E, H, k, x, ntok, x_stride, lg, ids, w);
  if (rc) goto done;
  for (uint32_t t = 0; t < ntok; t++)
    for (uint32_t r = 0; r < k; r++) {
      orc_job *j = &jobs[t * k + r];
      const int32_t e = ids[t * k + r];
      j->gate = L->gate[e], j->up = L->up[e], j->down = L->down[e];
      j->tok = t, j->w = w[t * k + r];
    }
  orc_shape sh = {L->gate_type, L->down_type, H, L->n_ff, L->swiglu_limit, 0};
  rc = orc_compute_many(&sh, jobs, ntok * k, ntok, x, x_stride, y, y_stride, nthreads);
  if (rc || !L->sh_gate) goto done;
  for (uint32_t t = 0; t < ntok; t++) {
    jobs[t].gate = L->sh_gate, jobs[t].up = L->sh_up, jobs[t].down = L->sh_down;
    jobs[t].tok = t, jobs[t].w = 1.0f;
  }
  orc_shape ss = {L->sh_gate_type, L->sh_down_type, H, L->n_ff, L->swiglu_limit, L->sh_up_type};
  rc = orc_compute_many(&ss, jobs, ntok, ntok, x, x_stride, s, H, nthreads);
  if (rc) goto done;
  for (uint32_t t = 0; t < ntok; t++) {
    const float gs = 1.0f / (1.0f + expf(-lg[(uint64_t)t * (E + 1) + E]));
    float *yt = y + t * y_stride;
    for (uint32_t i = 0; i < H; i++) yt[i] = yt[i] + gs * s[(uint64_t)t * H + i];
  }
done:
  if (!rc && ids_out) memcpy(ids_out, ids, sizeof(int32_t) * ntok * k);
  if (!rc && w_out) memcpy(w_out, w, sizeof(float) * ntok * k);
  free(lg), free(ids), free(w), free(jobs), free(s);
  return rc;
}

/* The block with some routed experts off the device (the hybrid: layer.cl:869-884): per token the resident experts'
 * outputs summed in rank order (compute_many on those jobs), + gs s, + the misses' sum (compute_many on the misses in
 * rank order, the CPU's answer), each sum rounded as it is added. resident: n_expert flags. */
int orc_moe_forward_resident(const orc_layer *L, const uint8_t *resident, const float *x, uint32_t ntok,
                             uint64_t x_stride, float *y, uint64_t y_stride, int nthreads) {
  const uint32_t E = L->n_expert, H = L->n_embd, k = L->n_used;
  if (ntok == 0) return 0;
  float *lg = (float *)malloc(sizeof(float) * ntok * (E + 1));
  int32_t *ids = (int32_t *)malloc(sizeof(int32_t) * ntok * k);
  float *w = (float *)malloc(sizeof(float) * ntok * k);
  orc_job *jobs = (orc_job *)malloc(sizeof(orc_job) * ntok * k);
  float *s = (float *)malloc(sizeof(float) * ntok * H), *cpu = (float *)malloc(sizeof(float) * ntok * H);
  orc_shape sh = {L->gate_type, L->down_type, H, L->n_ff, L->swiglu_limit, 0};
  int rc = orc_route(L->router, L->bias, E, H, k, x, ntok, x_stride, lg, ids, w);
  uint32_t n = 0;
  if (rc) goto done;
  for (int pass = 0; pass < 2; pass++) { /* 0: the resident jobs into y; 1: the misses into cpu */
    n = 0;
    for (uint32_t t = 0; t < ntok; t++)
      for (uint32_t r = 0; r < k; r++) {
        const int32_t e = ids[t * k + r];
        if ((resident[e] != 0) != (pass == 0)) continue;
        orc_job *j = &jobs[n++];
        j->gate = L->gate[e], j->up = L->up[e], j->down = L->down[e];
        j->tok = t, j->w = w[t * k + r];
      }
    rc = orc_compute_many(&sh, jobs, n, ntok, x, x_stride, pass ? cpu : y, pass ? H : y_stride, nthreads);
    if (rc) goto done;
  }
  if (L->sh_gate) {
    for (uint32_t t = 0; t < ntok; t++) {
      jobs[t].gate = L->sh_gate, jobs[t].up = L->sh_up, jobs[t].down = L->sh_down;
      jobs[t].tok = t, jobs[t].w = 1.0f;
    }
    orc_shape ss = {L->sh_gate_type, L->sh_down_type, H, L->n_ff, L->swiglu_limit, L->sh_up_type};
    rc = orc_compute_many(&ss, jobs, ntok, ntok, x, x_stride, s, H, nthreads);
    if (rc) goto done;
  }
  for (uint32_t t = 0; t < ntok; t++) {
    const float gs = 1.0f / (1.0f + expf(-lg[(uint64_t)t * (E + 1) + E]));
    uint32_t miss = 0;
    for (uint32_t r = 0; r < k; r++) miss += resident[ids[t * k + r]] == 0;
    float *yt = y + t * y_stride;
    for (uint32_t i = 0; i < H; i++) {
      if (L->sh_gate) yt[i] = yt[i] + gs * s[(uint64_t)t * H + i];
      if (miss) yt[i] = yt[i] + cpu[(uint64_t)t * H + i];
    }
  }
done:
  free(lg), free(ids), free(w), free(jobs), free(s), free(cpu);
  return rc;
}

/* ---------------------------------------------------------------------------------------------------------------
 * The hyper-connection mix and combine around the block (docs/spec/MODEL_LAYER.md 1.1-1.2: build_hc_mix and
 * build_hc_combine; the CPU ops ggml_compute_forward_rms_norm_f32 and the BF16 products, whose fp32 sums run in an
 * order of ggml's own, unpinned: here every BF16 product is exact and the products are summed in double, W_down's
 * and W_inject's rows in dot_tree_bf16's order, W_up's in k order, then rounded once). */

static inline float bf16r(float x) { return bf16_to_fp32(orc_fp32_to_bf16(x)); }
static inline float sigmoidf_(float z) { return 1.0f / (1.0f + expf(-z)); }

/* The decode kernel's order for a bf16 row of K values (a multiple of 512) against bf16(x): K in chunks of 512, lane
 * l of a chunk the values 8 l .. 8 l + 7 (a fused chain in k order from 0, each product exact); the 16 lanes of a
 * lane row r as ((P0 + P7) + (P3 + P4)) + ((P1 + P6) + (P2 + P5)), P_m = a_m + a_(15 - m); slot 4 w + r (wave w takes
 * chunks w, w + 4, ..) the chunks' sums in chunk order; the result the 16 slots added in order from 0. Where the
 * double sum is not exact (K of 10240 values of wide range), this fixes its rounding. */
static double dot_tree_bf16(const uint16_t *w, const float *x, uint32_t K) {
  const uint32_t nC = K / 512;
  double part[16] = {0};
  for (uint32_t c = 0; c < nC; c++) {
    const uint32_t wv = c % 4;
    for (uint32_t r = 0; r < 4; r++) {
      double a[16];
      for (uint32_t m = 0; m < 16; m++) {
        const uint32_t k0 = 512 * c + 8 * (16 * r + m);
        double acc = 0.0;
        for (uint32_t k = 0; k < 8; k++) acc += (double)bf16_to_fp32(w[k0 + k]) * (double)bf16r(x[k0 + k]);
        a[m] = acc;
      }
      double P[8];
      for (uint32_t m = 0; m < 8; m++) P[m] = a[m] + a[15 - m];
      const double S = ((P[0] + P[7]) + (P[3] + P[4])) + ((P[1] + P[6]) + (P[2] + P[5]));
      double *q = part + 4 * wv + r;
      *q = c < 4 ? S : *q + S;
    }
  }
  double s = 0.0;
  for (uint32_t i = 0; i < 16; i++) s += part[i];
  return s;
}

int orc_hc_pre(const float *R, uint32_t T, uint32_t H, uint32_t lr, const float *gamma, const uint16_t *w_down,
               const uint16_t *w_inj, const uint16_t *w_up, float *x, float *inject) {
  const uint64_t D = 4ull * H;
  float *n = (float *)malloc(sizeof(float) * D), *l = (float *)malloc(sizeof(float) * (lr ? lr : 1));
  if (!n || !l) return -1;
  for (uint32_t t = 0; t < T; t++) {
    const float *r = R + (uint64_t)t * D;
    for (uint32_t s = 0; s < 4; s++) { /* step 1: RMSNorm_1e-6(R_s) g_s, the squares summed in double */
      double ss = 0.0;
      for (uint32_t i = 0; i < H; i++) ss += (double)(r[s * H + i] * r[s * H + i]);
      const float mean = (float)(ss / (double)H);
      const float scale = 1.0f / sqrtf(mean + 1e-6f);
      for (uint32_t i = 0; i < H; i++) n[s * H + i] = (r[s * H + i] * scale) * gamma[s * H + i];
    }
    for (uint32_t j = 0; j < lr + 4; j++) { /* step 2: l = silu((W_down n) / 4); step 4: inject = W_inj n */
      const uint16_t *w = j < lr ? w_down + (uint64_t)j * D : w_inj + (uint64_t)(j - lr) * D;
      const float v = (float)dot_tree_bf16(w, n, (uint32_t)D);
      if (j < lr) {
        const float z = v * 0.25f;
        l[j] = z / (1.0f + expf(-z));
      } else {
        inject[(uint64_t)t * 4 + (j - lr)] = v;
      }
    }
    for (uint32_t i = 0; i < H; i++) { /* a = W_up l; step 3: x[i] = (sum_s n_s[i] sigma(a_s[i])) / 4 */
      float mix = 0.0f;
      for (uint32_t s = 0; s < 4; s++) {
        const uint16_t *w = w_up + ((uint64_t)s * H + i) * lr;
        double acc = 0.0;
        for (uint32_t k = 0; k < lr; k++) acc += (double)bf16_to_fp32(w[k]) * (double)bf16r(l[k]);
        mix = mix + n[s * H + i] * sigmoidf_((float)acc);
      }
      x[(uint64_t)t * H + i] = mix * 0.25f;
    }
  }
  free(n);
  free(l);
  return 0;
}

void orc_hc_post(float *R, uint32_t T, uint32_t H, const float *inject, const float *y) {
  for (uint32_t t = 0; t < T; t++)
    for (uint32_t s = 0; s < 4; s++) {
      const float w = 2.0f * sigmoidf_(inject[(uint64_t)t * 4 + s] * 0.25f);
      float *r = R + ((uint64_t)t * 4 + s) * H;
      for (uint32_t i = 0; i < H; i++) r[i] = r[i] + w * y[(uint64_t)t * H + i];
    }
}
