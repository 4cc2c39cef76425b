/* TEST INFRASTRUCTURE - the CPU baseline of bench.py: the block as the reference's CPU expert path computes it
 * (core/cpu/experts.cpp:152-284, CpuExperts::compute_many; the router of docs/spec/MODEL_LAYER.md:414-425), with the
 * oracle's every rounding (oracle.h, ORACLE ORDER), made fast:
 *   - the integer part of each block dot product with SIMD (AVX-512BW when the CPU has it, else AVX2): unsigned x
 *     signed byte products (vpmaddubsw), the block scales applied by vpmaddwd, then one horizontal sum; a sign that
 *     belongs to the weight moves to the activation byte (q8 codes lie in [-127, 127]). Integer sums are exact, so
 *     the order inside them is free;
 *   - the fp32 steps per block or unit exactly as oracle.c writes them (this file is built with -ffp-contract=off),
 *     units of a row added in sequence;
 *   - each weight unit decoded once for all the jobs (tokens) of its expert;
 *   - router logits with the expert rows as SIMD lanes, each lane adding its products in k order in double (the
 *     oracle's sum, lane by lane);
 *   - OpenMP over (expert, row) tasks, as orc_compute_many.
 * Checked bit for bit against orc_moe_forward in tests/test_cpu_fast.py. Only bench.py's cpu_baseline leg and the
 * tests load it. */
#include <immintrin.h>
#include <math.h>
#include <omp.h>
#include <stdlib.h>
#include <string.h>

#include "oracle.h"

#define QT_Q8_0 8
#define QT_Q4_K 12
#define QT_Q8_K 15
#define QT_IQ3_S 21
#define QK 256

static int g_isa = -1; /* 2: AVX-512BW, 1: AVX2 */
static uint32_t g_grid[512];

static void fast_init(void) {
  if (g_isa >= 0) return;
  orc_iq3s_grid(g_grid);
  __builtin_cpu_init();
  g_isa = __builtin_cpu_supports("avx512bw") && __builtin_cpu_supports("avx512vl") ? 2 : 1;
  const char *force = getenv("C0VEN_CPU_ISA");  /* "avx2": the AVX2 paths even where AVX-512 is there (tests) */
  if (force && strcmp(force, "avx2") == 0) g_isa = 1;
}

const char *orc_fast_isa(void) {
  fast_init();
  return g_isa == 2 ? "avx512bw" : "avx2";
}

static inline float h2f(const uint8_t *p) { return orc_fp16_to_fp32((uint16_t)(p[0] | (p[1] << 8))); }

static uint32_t act_type_of(uint32_t t) { return t == QT_Q8_0 ? QT_Q8_0 : QT_Q8_K; }
static uint64_t act_bytes(uint32_t act, uint64_t n) { return act == QT_Q8_0 ? n / 32 * 34 : n / QK * 292; }
static uint64_t row_bytes(uint32_t t, uint64_t n) {
  return t == QT_Q8_0 ? n / 32 * 34 : t == QT_Q4_K ? n / QK * 144 : n / QK * 110;
}

/* ---------------------------------------------------------------------------------------------------------------
 * A weight unit (256 values) prepared once for every job: 256 unsigned magnitudes, the weight signs as a 256-bit
 * mask, the 16-bit scale of each 32-value sub-block, and the unit's fp32 scales. */
typedef struct {
  uint8_t mag[256] __attribute__((aligned(64)));
  uint64_t neg[4];  /* bit v: value v negative */
  int16_t sc[8];    /* sub-block scales (Q4_K sc, IQ3_S 1 + 2 s, Q8_0 1) */
  int m[8];         /* Q4_K minima */
  float d, dmin;    /* Q4_K d, dmin; IQ3_S d */
  float dq[8];      /* Q8_0 block scales */
} Unit;

__attribute__((target("avx2"))) static void prep_q4k(const uint8_t *b, Unit *u) {
  u->d = h2f(b), u->dmin = h2f(b + 2);
  const uint8_t *q = b + 4;
  for (int j = 0; j < 8; j++) {
    int sc, m;
    if (j < 4) {
      sc = q[j] & 63, m = q[j + 4] & 63;
    } else {
      sc = (q[j + 4] & 0xF) | ((q[j - 4] >> 6) << 4), m = (q[j + 4] >> 4) | ((q[j] >> 6) << 4);
    }
    u->sc[j] = (int16_t)sc, u->m[j] = m;
  }
  const uint8_t *qs = b + 16;
  const __m256i lo4 = _mm256_set1_epi8(0x0F);
  for (int c = 0; c < 4; c++) {  /* sub-block 2 c: low nibbles; 2 c + 1: high nibbles */
    const __m256i v = _mm256_loadu_si256((const __m256i *)(qs + 32 * c));
    _mm256_store_si256((__m256i *)(u->mag + 64 * c), _mm256_and_si256(v, lo4));
    _mm256_store_si256((__m256i *)(u->mag + 64 * c + 32), _mm256_and_si256(_mm256_srli_epi16(v, 4), lo4));
  }
  u->neg[0] = u->neg[1] = u->neg[2] = u->neg[3] = 0;
}

__attribute__((target("avx2"))) static void prep_iq3s(const uint8_t *b, Unit *u) {
  u->d = h2f(b);
  const uint8_t *qs = b + 2, *qh = b + 66, *signs = b + 74, *scales = b + 106;
  const __m256i kbit = _mm256_setr_epi32(1, 2, 4, 8, 16, 32, 64, 128);
  for (int ib = 0; ib < 8; ib++) {
    u->sc[ib] = (int16_t)(1 + 2 * ((scales[ib / 2] >> (4 * (ib % 2))) & 15));
    /* the 8 groups' 9-bit grid indices: qs byte | (bit k of qh) << 8, then one gather of their grid words */
    const __m256i lo = _mm256_cvtepu8_epi32(_mm_loadl_epi64((const __m128i *)(qs + 8 * ib)));
    const __m256i hb = _mm256_and_si256(_mm256_set1_epi32(qh[ib]), kbit);
    const __m256i idx = _mm256_or_si256(lo, _mm256_slli_epi32(_mm256_min_epu32(hb, _mm256_set1_epi32(1)), 8));
    _mm256_store_si256((__m256i *)(u->mag + 32 * ib), _mm256_i32gather_epi32((const int *)g_grid, idx, 4));
  }
  memcpy(u->neg, signs, 32);
}

__attribute__((target("avx2"))) static void prep_q8_0(const uint8_t *b, Unit *u) {
  u->neg[0] = u->neg[1] = u->neg[2] = u->neg[3] = 0;
  for (int j = 0; j < 8; j++) {
    const uint8_t *blk = b + 34 * j;
    u->dq[j] = h2f(blk);
    u->sc[j] = 1;
    const __m256i v = _mm256_loadu_si256((const __m256i *)(blk + 2));
    _mm256_store_si256((__m256i *)(u->mag + 32 * j), _mm256_abs_epi8(v));  /* -128 does not occur in q8_0 weights */
    u->neg[j / 2] |= (uint64_t)(uint32_t)_mm256_movemask_epi8(v) << (32 * (j % 2));
  }
}

__attribute__((target("avx2"))) static inline int32_t hsum256(__m256i v) {
  __m128i x = _mm_add_epi32(_mm256_castsi256_si128(v), _mm256_extracti128_si256(v, 1));
  x = _mm_add_epi32(x, _mm_shuffle_epi32(x, 0x4e));
  x = _mm_add_epi32(x, _mm_shuffle_epi32(x, 0xb1));
  return _mm_cvtsi128_si32(x);
}

/* sum over the 8 sub-blocks j of sc[j] * sum_{v in j} mag[v] * (neg[v] ? -a[v] : a[v]); per sub-block sums in s[] when
 * s is not null (Q8_0). */
__attribute__((target("avx512f,avx512bw,avx512vl"))) static int32_t idot_512(const Unit *u, const int8_t *a, int32_t *s) {
  __m512i acc = _mm512_setzero_si512();
  for (int c = 0; c < 4; c++) {
    const __m512i m = _mm512_load_si512((const void *)(u->mag + 64 * c));
    __m512i av = _mm512_loadu_si512((const void *)(a + 64 * c));
    av = _mm512_mask_sub_epi8(av, (__mmask64)u->neg[c], _mm512_setzero_si512(), av);
    const __m512i p16 = _mm512_maddubs_epi16(m, av);
    const __m512i scv = _mm512_inserti64x4(_mm512_castsi256_si512(_mm256_set1_epi16(u->sc[2 * c])),
                                           _mm256_set1_epi16(u->sc[2 * c + 1]), 1);
    const __m512i p32 = _mm512_madd_epi16(p16, scv);
    if (s) {
      s[2 * c] = hsum256(_mm512_castsi512_si256(p32));
      s[2 * c + 1] = hsum256(_mm512_extracti64x4_epi64(p32, 1));
    }
    acc = _mm512_add_epi32(acc, p32);
  }
  return _mm512_reduce_add_epi32(acc);
}

__attribute__((target("avx2"))) static int32_t idot_256(const Unit *u, const int8_t *a, int32_t *s) {
  int32_t tot = 0;
  for (int j = 0; j < 8; j++) {
    const __m256i m = _mm256_load_si256((const __m256i *)(u->mag + 32 * j));
    __m256i av = _mm256_loadu_si256((const __m256i *)(a + 32 * j));
    const uint32_t bits = (uint32_t)(u->neg[j / 2] >> (32 * (j % 2)));
    /* the 32 sign bits as a byte mask: byte b takes bit b */
    const __m256i sel = _mm256_setr_epi8(0, 0, 0, 0, 0, 0, 0, 0, 1, 1, 1, 1, 1, 1, 1, 1, 2, 2, 2, 2, 2, 2, 2, 2, 3, 3, 3,
                                         3, 3, 3, 3, 3);
    const __m256i bitsel = _mm256_set1_epi64x((long long)0x8040201008040201ull);
    const __m256i bb = _mm256_shuffle_epi8(_mm256_set1_epi32((int)bits), sel);
    const __m256i negm = _mm256_cmpeq_epi8(_mm256_and_si256(bb, bitsel), bitsel);
    av = _mm256_sub_epi8(_mm256_xor_si256(av, negm), negm);
    const __m256i p16 = _mm256_maddubs_epi16(m, av);
    const int32_t sj = hsum256(_mm256_madd_epi16(p16, _mm256_set1_epi16(1)));
    if (s) s[j] = sj;
    tot += u->sc[j] * sj;
  }
  return tot;
}

static inline int32_t idot(const Unit *u, const int8_t *a, int32_t *s) {
  return g_isa == 2 ? idot_512(u, a, s) : idot_256(u, a, s);
}

/* The unit's fp32 term against activation unit a, as oracle.c's term_* / dot_row compute it. */
static inline float unit_term(uint32_t type, const Unit *u, const uint8_t *a) {
  if (type == QT_Q8_0) {
    /* eight q8_0 blocks (34 B each): (d_w d_a) dot per block, pairwise tree */
    int8_t codes[256] __attribute__((aligned(64)));
    for (int j = 0; j < 8; j++) memcpy(codes + 32 * j, a + 34 * j + 2, 32);
    int32_t s[8];
    (void)idot(u, codes, s);
    float t[8];
    for (int j = 0; j < 8; j++) {
      const float d = u->dq[j] * h2f(a + 34 * j);
      t[j] = d * (float)s[j];
    }
    return ((t[0] + t[1]) + (t[2] + t[3])) + ((t[4] + t[5]) + (t[6] + t[7]));
  }
  float ad;
  memcpy(&ad, a, 4);
  const int8_t *q8 = (const int8_t *)(a + 4);
  const int32_t isum = idot(u, q8, NULL);
  if (type == QT_Q4_K) {
    int16_t bs[16];
    memcpy(bs, a + 260, 32);
    int32_t imin = 0;
    for (int j = 0; j < 8; j++) imin += u->m[j] * (bs[2 * j] + bs[2 * j + 1]);
    const float d = u->d * ad, dm = u->dmin * ad;
    const float pm = dm * (float)imin;
    return fmaf(d, (float)isum, -pm);
  }
  const float d = u->d * ad;
  return d * (float)isum;
}

static void prep(uint32_t type, const uint8_t *w, Unit *u) {
  if (type == QT_Q4_K)
    prep_q4k(w, u);
  else if (type == QT_IQ3_S)
    prep_iq3s(w, u);
  else
    prep_q8_0(w, u);
}

static uint32_t unit_bytes_w(uint32_t t) { return t == QT_Q8_0 ? 8 * 34 : t == QT_Q4_K ? 144 : 110; }
static uint32_t unit_bytes_a(uint32_t act) { return act == QT_Q8_0 ? 8 * 34 : 292; }

/* Row r of a matrix against the activation rows of n jobs: out[j] = the row's dot with act[idx[j]], units in
 * sequence. */
static void row_dots(uint32_t type, const uint8_t *row, uint32_t U, const uint8_t *act, uint64_t act_stride,
                     const uint32_t *idx, uint32_t n, float *out) {
  const uint32_t uw = unit_bytes_w(type), ua = unit_bytes_a(act_type_of(type));
  Unit u;
  for (uint32_t j = 0; j < n; j++) out[j] = 0.0f;
  for (uint32_t k = 0; k < U; k++) {
    prep(type, row + (uint64_t)k * uw, &u);
    for (uint32_t j = 0; j < n; j++) out[j] = out[j] + unit_term(type, &u, act + idx[j] * act_stride + (uint64_t)k * ua);
  }
}

static inline float swiglu_one(float g, float u, float limit) {
  if (limit > 0.0f) {
    g = fminf(g, limit);
    u = u < -limit ? -limit : (u > limit ? limit : u);
  }
  return g / (1.0f + expf(-g)) * u;
}

/* CpuExperts::compute_many with the oracle's bits (orc_compute_many's arithmetic, job for job). */
static int fast_compute_many(const orc_shape *s, const orc_job *jobs, uint32_t njobs, uint32_t ntok, const float *x,
                             uint64_t x_stride, float *y, uint64_t y_stride, int nthreads) {
  const uint32_t E = s->n_embd, F = s->n_ff;
  for (uint32_t t = 0; t < ntok; t++) memset(y + t * y_stride, 0, sizeof(float) * E);
  if (njobs == 0) return 0;
  if (E % QK || F % QK) return -1;
  if (s->up_type && s->up_type != s->gate_type) return -1;
  for (int m = 0; m < 2; m++) { /* the config types: Q8_0, Q4_K, IQ3_S */
    const uint32_t t = m ? s->down_type : s->gate_type;
    if (t != QT_Q8_0 && t != QT_Q4_K && t != QT_IQ3_S) return -1;
  }
  const uint32_t ga = act_type_of(s->gate_type), da = act_type_of(s->down_type);
  const uint64_t xq_bytes = act_bytes(ga, E), hq_bytes = act_bytes(da, F);
  const uint64_t grow = row_bytes(s->gate_type, E), drow = row_bytes(s->down_type, F);
  uint8_t *xq = (uint8_t *)malloc(ntok * xq_bytes), *hq = (uint8_t *)malloc(njobs * hq_bytes);
  float *h = (float *)malloc(sizeof(float) * njobs * F), *out = (float *)malloc(sizeof(float) * njobs * E);
  uint32_t *dj = (uint32_t *)malloc(sizeof(uint32_t) * njobs), *dstart = (uint32_t *)malloc(sizeof(uint32_t) * (njobs + 1));
  uint32_t *tok = (uint32_t *)malloc(sizeof(uint32_t) * njobs), *jid = (uint32_t *)malloc(sizeof(uint32_t) * njobs);
  uint8_t *taken = (uint8_t *)calloc(njobs, 1);
  for (uint32_t t = 0; t < ntok; t++) orc_quantize_act(ga, x + t * x_stride, xq + t * xq_bytes, E);
  uint32_t nd = 0, nj = 0;
  for (uint32_t j = 0; j < njobs; j++) {
    if (taken[j]) continue;
    dstart[nd++] = nj;
    for (uint32_t i = j; i < njobs; i++)
      if (!taken[i] && jobs[i].gate == jobs[j].gate) taken[i] = 1, dj[nj++] = i;
  }
  dstart[nd] = nj;
  for (uint32_t i = 0; i < njobs; i++) tok[i] = jobs[dj[i]].tok, jid[i] = i;
  const int64_t tasks_gu = (int64_t)nd * F;
#pragma omp parallel num_threads(nthreads)
  {
    float *g = (float *)malloc(sizeof(float) * njobs), *u = (float *)malloc(sizeof(float) * njobs);
#pragma omp for schedule(dynamic, 16)
    for (int64_t task = 0; task < tasks_gu; task++) {
      const uint32_t d = (uint32_t)(task / F), r = (uint32_t)(task % F), n = dstart[d + 1] - dstart[d];
      const orc_job *j0 = &jobs[dj[dstart[d]]];
      row_dots(s->gate_type, j0->gate + r * grow, E / QK, xq, xq_bytes, tok + dstart[d], n, g);
      row_dots(s->gate_type, j0->up + r * grow, E / QK, xq, xq_bytes, tok + dstart[d], n, u);
      for (uint32_t i = 0; i < n; i++) h[(uint64_t)dj[dstart[d] + i] * F + r] = swiglu_one(g[i], u[i], s->swiglu_limit);
    }
    free(g), free(u);
  }
  for (uint32_t j = 0; j < njobs; j++) orc_quantize_act(da, h + (uint64_t)j * F, hq + j * hq_bytes, F);
  const int64_t tasks_d = (int64_t)nd * E;
#pragma omp parallel num_threads(nthreads)
  {
    float *o = (float *)malloc(sizeof(float) * njobs);
#pragma omp for schedule(dynamic, 16)
    for (int64_t task = 0; task < tasks_d; task++) {
      const uint32_t d = (uint32_t)(task / E), r = (uint32_t)(task % E), n = dstart[d + 1] - dstart[d];
      const orc_job *j0 = &jobs[dj[dstart[d]]];
      row_dots(s->down_type, j0->down + r * drow, F / QK, hq, hq_bytes, dj + dstart[d], n, o);
      for (uint32_t i = 0; i < n; i++) out[(uint64_t)dj[dstart[d] + i] * E + r] = o[i];
    }
    free(o);
  }
  for (uint32_t j = 0; j < njobs; j++) {
    float *yt = y + jobs[j].tok * y_stride;
    const float w = jobs[j].w;
    for (uint32_t r = 0; r < E; r++) yt[r] = yt[r] + w * out[(uint64_t)j * E + r];
  }
  free(xq), free(hq), free(h), free(out), free(dj), free(dstart), free(tok), free(jid), free(taken);
  return 0;
}

/* ---------------------------------------------------------------------------------------------------------------
 * Router logits: the rows (experts) as lanes, each adding its exact fp32 products in double in k order. The router is
 * transposed to k-major fp32 once per router pointer. */
static const uint16_t *g_rt_src = NULL;
static float *g_rt = NULL; /* H x R, R = E + 1 rounded up to 16 */
static uint32_t g_rt_R = 0;

static void router_t(const uint16_t *router, uint32_t E, uint32_t H) {
  if (g_rt_src == router && g_rt) return;
  free(g_rt);
  const uint32_t R = (E + 1 + 15) / 16 * 16;
  g_rt = (float *)calloc((uint64_t)H * R, sizeof(float));
  for (uint32_t e = 0; e <= E; e++)
    for (uint32_t k = 0; k < H; k++) {
      const uint32_t b = (uint32_t)router[(uint64_t)e * H + k] << 16;
      memcpy(&g_rt[(uint64_t)k * R + e], &b, 4);
    }
  g_rt_src = router, g_rt_R = R;
}

__attribute__((target("avx512f"))) static void logits_512(const float *xb, uint32_t H, uint32_t R, float *lg) {
  for (uint32_t e0 = 0; e0 < R; e0 += 64) {
    __m512d acc[8];
    for (int i = 0; i < 8; i++) acc[i] = _mm512_setzero_pd();
    const uint32_t ne = R - e0 < 64 ? R - e0 : 64;
    for (uint32_t k = 0; k < H; k++) {
      const __m512 xv = _mm512_set1_ps(xb[k]);
      const float *wr = g_rt + (uint64_t)k * R + e0;
      for (uint32_t i = 0; i < ne / 16; i++) {
        const __m512 p = _mm512_mul_ps(_mm512_loadu_ps(wr + 16 * i), xv); /* exact: bf16 x bf16 */
        acc[2 * i] = _mm512_add_pd(acc[2 * i], _mm512_cvtps_pd(_mm512_castps512_ps256(p)));
        acc[2 * i + 1] = _mm512_add_pd(acc[2 * i + 1], _mm512_cvtps_pd(_mm256_castpd_ps(_mm512_extractf64x4_pd(_mm512_castps_pd(p), 1))));
      }
    }
    for (uint32_t i = 0; i < ne / 8; i++) {
      double t[8];
      _mm512_storeu_pd(t, acc[i]);
      for (int q = 0; q < 8; q++) lg[e0 + 8 * i + q] = (float)t[q];
    }
  }
}

__attribute__((target("avx2"))) static void logits_256(const float *xb, uint32_t H, uint32_t R, float *lg) {
  for (uint32_t e0 = 0; e0 < R; e0 += 16) {
    __m256d acc[4];
    for (int i = 0; i < 4; i++) acc[i] = _mm256_setzero_pd();
    for (uint32_t k = 0; k < H; k++) {
      const __m256 xv = _mm256_set1_ps(xb[k]);
      const float *wr = g_rt + (uint64_t)k * R + e0;
      for (int i = 0; i < 2; i++) {
        const __m256 p = _mm256_mul_ps(_mm256_loadu_ps(wr + 8 * i), xv);
        acc[2 * i] = _mm256_add_pd(acc[2 * i], _mm256_cvtps_pd(_mm256_castps256_ps128(p)));
        acc[2 * i + 1] = _mm256_add_pd(acc[2 * i + 1], _mm256_cvtps_pd(_mm256_extractf128_ps(p, 1)));
      }
    }
    for (int i = 0; i < 4; i++) {
      double t[4];
      _mm256_storeu_pd(t, acc[i]);
      for (int q = 0; q < 4; q++) lg[e0 + 4 * i + q] = (float)t[q];
    }
  }
}

int orc_fast_moe_forward(const orc_layer *L, const float *x, uint32_t ntok, uint64_t x_stride, float *y,
                         uint64_t y_stride, int32_t *ids_out, float *w_out, int nthreads) {
  fast_init();
  const uint32_t E = L->n_expert, H = L->n_embd, k = L->n_used;
  if (ntok == 0) return 0;
  if (nthreads <= 0) nthreads = 1;
  router_t(L->router, E, H);
  const uint32_t R = g_rt_R;
  float *lg = (float *)malloc(sizeof(float) * ntok * R);
  int32_t *ids = (int32_t *)malloc(sizeof(int32_t) * ntok * k);
  float *w = (float *)malloc(sizeof(float) * ntok * k);
  orc_job *jobs = (orc_job *)malloc(sizeof(orc_job) * ntok * (k > 1 ? k : 1));
  float *s = (float *)malloc(sizeof(float) * ntok * H);
  int rc = 0;
#pragma omp parallel for num_threads(nthreads) schedule(dynamic, 1)
  for (uint32_t t = 0; t < ntok; t++) {
    float *xb = (float *)malloc(sizeof(float) * H), *lt = lg + (uint64_t)t * R;
    for (uint32_t i = 0; i < H; i++) {
      const uint32_t b = (uint32_t)orc_fp32_to_bf16(x[t * x_stride + i]) << 16;
      memcpy(&xb[i], &b, 4);
    }
    if (g_isa == 2)
      logits_512(xb, H, R, lt);
    else
      logits_256(xb, H, R, lt);
    if (L->bias)
      for (uint32_t e = 0; e < E; e++) lt[e] = lt[e] + L->bias[e];
    orc_topk_logits(lt, E, k, ids + (uint64_t)t * k, w + (uint64_t)t * k);
    free(xb);
  }
  for (uint32_t t = 0; t < ntok; t++)
    for (uint32_t r = 0; r < k; r++) {
      orc_job *j = &jobs[t * k + r];
      const int32_t e = ids[t * k + r];
      j->gate = L->gate[e], j->up = L->up[e], j->down = L->down[e];
      j->tok = t, j->w = w[t * k + r];
    }
  orc_shape sh = {L->gate_type, L->down_type, H, L->n_ff, L->swiglu_limit, 0};
  rc = fast_compute_many(&sh, jobs, ntok * k, ntok, x, x_stride, y, y_stride, nthreads);
  if (!rc && L->sh_gate) {
    for (uint32_t t = 0; t < ntok; t++) {
      jobs[t].gate = L->sh_gate, jobs[t].up = L->sh_up, jobs[t].down = L->sh_down;
      jobs[t].tok = t, jobs[t].w = 1.0f;
    }
    orc_shape ss = {L->sh_gate_type, L->sh_down_type, H, L->n_ff, L->swiglu_limit, L->sh_up_type};
    rc = fast_compute_many(&ss, jobs, ntok, ntok, x, x_stride, s, H, nthreads);
    if (!rc)
      for (uint32_t t = 0; t < ntok; t++) {
        const float gs = 1.0f / (1.0f + expf(-lg[(uint64_t)t * R + E]));
        float *yt = y + t * y_stride;
        for (uint32_t i = 0; i < H; i++) yt[i] = yt[i] + gs * s[(uint64_t)t * H + i];
      }
  }
  if (!rc && ids_out) memcpy(ids_out, ids, sizeof(int32_t) * ntok * k);
  if (!rc && w_out) memcpy(w_out, w, sizeof(float) * ntok * k);
  free(lg), free(ids), free(w), free(jobs), free(s);
  return rc;
}
