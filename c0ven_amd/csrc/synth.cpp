// Seeded synthetic inputs and the weight quantisers (host). The configs' weights are N(0, sigma) fp32 values
// quantised to the expert types; every machine draws the same values from (seed, stream, index).
#include <algorithm>
#include <cmath>
#include <cstring>
#include <mutex>
#include <thread>
#include <vector>

#include "../../include/c0ven_moe.h"
#include "iq3s_grid.h"

namespace c0ven {
namespace {

inline uint64_t splitmix64(uint64_t x) {
  x += 0x9e3779b97f4a7c15ull;
  x = (x ^ (x >> 30)) * 0xbf58476d1ce4e5b9ull;
  x = (x ^ (x >> 27)) * 0x94d049bb133111ebull;
  return x ^ (x >> 31);
}

// Normal i of (seed, stream): Box-Muller on two counter-based uniforms per pair of values.
struct Normal {
  uint64_t key;
  Normal(uint64_t seed, uint64_t stream) : key(splitmix64(seed ^ splitmix64(stream * 0x2545f4914f6cdd1dull + 1))) {}
  void pair(uint64_t p, double &z0, double &z1) const {
    const uint64_t r1 = splitmix64(key + 2 * p), r2 = splitmix64(key + 2 * p + 1);
    const double u1 = ((double)(r1 >> 11) + 1.0) * 0x1p-53, u2 = (double)(r2 >> 11) * 0x1p-53;
    const double rad = std::sqrt(-2.0 * std::log(u1)), th = 6.283185307179586 * u2;
    z0 = rad * std::cos(th);
    z1 = rad * std::sin(th);
  }
  void fill(float sigma, float *out, uint64_t i0, uint64_t n) const {
    for (uint64_t i = i0; i < i0 + n; i++) {
      double z0, z1;
      pair(i / 2, z0, z1);
      out[i - i0] = (float)((i % 2 ? z1 : z0) * (double)sigma);
    }
  }
};

int threads_for(int nthreads) {
  if (nthreads > 0) return nthreads;
  const unsigned hc = std::thread::hardware_concurrency();
  return hc ? (int)std::min(hc, 64u) : 1;
}

template <typename F>
void parallel_for(uint64_t n, int nthreads, F f) {
  const int nt = (int)std::min<uint64_t>((uint64_t)threads_for(nthreads), std::max<uint64_t>(n, 1));
  if (nt <= 1) {
    for (uint64_t i = 0; i < n; i++) f(i);
    return;
  }
  std::vector<std::thread> th;
  for (int t = 0; t < nt; t++)
    th.emplace_back([=, &f] {
      for (uint64_t i = n * t / nt; i < n * (t + 1) / nt; i++) f(i);
    });
  for (auto &x : th) x.join();
}

inline uint16_t fp16_bits(float f) {
  _Float16 h = (_Float16)f;  // round to nearest even
  uint16_t b;
  std::memcpy(&b, &h, 2);
  return b;
}
inline float fp16_value(uint16_t b) {
  _Float16 h;
  std::memcpy(&h, &b, 2);
  return (float)h;
}
inline int nearest(float v) { return (int)std::nearbyint(v); }

// ggml's quantize_row_q8_0_ref: d = amax / 127, q = round(x / d) (half away from zero), d stored as f16.
void quant_q8_0(const float *x, uint8_t *y, uint32_t n) {
  for (uint32_t b = 0; b < n / 32; b++, x += 32, y += 34) {
    float amax = 0.0f;
    for (int j = 0; j < 32; j++) amax = std::max(amax, std::fabs(x[j]));
    const float d = amax / 127.0f, id = d != 0.0f ? 1.0f / d : 0.0f;
    const uint16_t dh = fp16_bits(d);
    std::memcpy(y, &dh, 2);
    for (int j = 0; j < 32; j++) y[2 + j] = (uint8_t)(int8_t)std::round(x[j] * id);
  }
}

// Q4_K: per sub-block of 32 the range [min(lo, 0), hi] in 15 steps, the steps and minimums as 6-bit multiples of
// their largest / 63, codes rounded to nearest with the rounded scales. Valid blocks, but not ggml's
// make_qkx2_quants search.
void quant_q4_K(const float *x, uint8_t *y, uint32_t n) {
  for (uint32_t b = 0; b < n / 256; b++, x += 256, y += 144) {
    float step[8], mins[8];
    for (int j = 0; j < 8; j++) {
      float lo = 0.0f, hi = 0.0f;
      for (int i = 0; i < 32; i++) lo = std::min(lo, x[32 * j + i]), hi = std::max(hi, x[32 * j + i]);
      mins[j] = -lo;
      step[j] = (hi - lo) / 15.0f;
    }
    const float smax = *std::max_element(step, step + 8), mmax = *std::max_element(mins, mins + 8);
    const uint16_t dh = fp16_bits(smax / 63.0f), mh = fp16_bits(mmax / 63.0f);
    const float d = fp16_value(dh), dmin = fp16_value(mh);
    int sc[8], m[8];
    for (int j = 0; j < 8; j++) {
      sc[j] = d > 0.0f ? std::clamp(nearest(step[j] / d), 0, 63) : 0;
      m[j] = dmin > 0.0f ? std::clamp(nearest(mins[j] / dmin), 0, 63) : 0;
      if (step[j] > 0.0f && sc[j] == 0) sc[j] = 1;
    }
    std::memcpy(y, &dh, 2);
    std::memcpy(y + 2, &mh, 2);
    uint8_t *s = y + 4;
    for (int j = 0; j < 4; j++) {
      s[j] = (uint8_t)((sc[j] & 63) | ((sc[j + 4] >> 4) << 6));
      s[j + 4] = (uint8_t)((m[j] & 63) | ((m[j + 4] >> 4) << 6));
      s[j + 8] = (uint8_t)((sc[j + 4] & 15) | ((m[j + 4] & 15) << 4));
    }
    uint8_t q[256];
    for (int j = 0; j < 8; j++) {
      const float dj = d * (float)sc[j], mj = dmin * (float)m[j];
      for (int i = 0; i < 32; i++) q[32 * j + i] = dj > 0.0f ? (uint8_t)std::clamp(nearest((x[32 * j + i] + mj) / dj), 0, 15) : 0;
    }
    for (int c = 0; c < 4; c++)
      for (int l = 0; l < 32; l++) y[16 + 32 * c + l] = (uint8_t)(q[64 * c + l] | (q[64 * c + 32 + l] << 4));
  }
}

// For each point of the 8^4 lattice of magnitude levels (2 l + 1), the nearest IQ3_S grid entry (squared distance,
// ties to the lower entry).
const std::vector<uint16_t> &iq3s_nearest() {
  static const std::vector<uint16_t> map = [] {
    std::vector<uint16_t> m(4096);
    for (uint32_t c = 0; c < 4096; c++) {
      int best = 0, bd = 1 << 30;
      for (int g = 0; g < 512; g++) {
        int dd = 0;
        for (int j = 0; j < 4; j++) {
          const int a = 2 * (int)((c >> (3 * j)) & 7) + 1, v = (int)((kIq3sGridHost[g] >> (8 * j)) & 0xff);
          dd += (a - v) * (a - v);
        }
        if (dd < bd) bd = dd, best = g;
      }
      m[c] = (uint16_t)best;
    }
    return m;
  }();
  return map;
}

// IQ3_S: per sub-block of 32 a step amax / 15 as d (1 + 2 s), d = the largest step / 31; each group of four
// magnitudes to its nearest lattice levels, then to the nearest grid entry; the signs stored plainly. Valid blocks,
// not ggml's quantize_row_iq3_s search.
void quant_iq3_s(const float *x, uint8_t *y, uint32_t n) {
  const std::vector<uint16_t> &near = iq3s_nearest();
  for (uint32_t b = 0; b < n / 256; b++, x += 256, y += 110) {
    std::memset(y, 0, 110);
    float step[8];
    for (int j = 0; j < 8; j++) {
      float a = 0.0f;
      for (int i = 0; i < 32; i++) a = std::max(a, std::fabs(x[32 * j + i]));
      step[j] = a / 15.0f;
    }
    const float smax = *std::max_element(step, step + 8);
    const uint16_t dh = fp16_bits(smax / 31.0f);
    const float d = fp16_value(dh);
    std::memcpy(y, &dh, 2);
    if (d <= 0.0f) continue;
    uint8_t *qs = y + 2, *qh = y + 66, *signs = y + 74, *scales = y + 106;
    for (int ib = 0; ib < 8; ib++) {
      const int s = std::clamp(nearest((step[ib] / d - 1.0f) / 2.0f), 0, 15);
      scales[ib / 2] |= (uint8_t)(s << (4 * (ib % 2)));
      const float db = d * (float)(1 + 2 * s);
      for (int k = 0; k < 8; k++) {
        uint32_t code = 0;
        for (int j = 0; j < 4; j++) {
          const float v = x[32 * ib + 4 * k + j];
          const int l = std::clamp(nearest((std::fabs(v) / db - 1.0f) / 2.0f), 0, 7);
          code |= (uint32_t)l << (3 * j);
          if (v < 0.0f) signs[4 * ib + (4 * k + j) / 8] |= (uint8_t)(1u << ((4 * k + j) % 8));
        }
        const uint32_t g = near[code];
        qs[8 * ib + k] = (uint8_t)(g & 0xff);
        qh[ib] |= (uint8_t)(((g >> 8) & 1u) << k);
      }
    }
  }
}

// The caller's iq2s_grid and iq3xxs_grid (moe_synth_set_codebooks), and for each point of their magnitude-level
// lattices (IQ3_XXS: 8 levels 4, 12, .., 52, 62 for 4 values; IQ2_S: 3 levels 8, 25, 43 for 8 values) the nearest
// entry (squared distance, ties to the lower entry).
struct CodebookMaps {
  std::vector<uint64_t> iq2s;
  std::vector<uint32_t> iq3xxs;
  std::vector<uint16_t> near2, near3;
};
std::mutex g_cb_mu;
CodebookMaps *g_cb = nullptr;  // set once per call of moe_synth_set_codebooks; kept until the process ends

constexpr int kIq3xxsLevel[8] = {4, 12, 20, 28, 36, 44, 52, 62};
constexpr int kIq2sLevel[3] = {8, 25, 43};

CodebookMaps *make_maps(const uint8_t *qgrid) {
  auto *m = new CodebookMaps;
  m->iq2s.resize(1024);
  m->iq3xxs.resize(256);
  std::memcpy(m->iq2s.data(), qgrid + QGRID_IQ2S, 8192);
  std::memcpy(m->iq3xxs.data(), qgrid + QGRID_IQ3XXS, 1024);
  m->near3.resize(4096);
  for (uint32_t c = 0; c < 4096; c++) {
    int best = 0, bd = 1 << 30;
    for (int g = 0; g < 256; g++) {
      int dd = 0;
      for (int j = 0; j < 4; j++) {
        const int a = kIq3xxsLevel[(c >> (3 * j)) & 7], v = (int)((m->iq3xxs[g] >> (8 * j)) & 0xff);
        dd += (a - v) * (a - v);
      }
      if (dd < bd) bd = dd, best = g;
    }
    m->near3[c] = (uint16_t)best;
  }
  m->near2.resize(6561);
  for (uint32_t c = 0; c < 6561; c++) {
    int best = 0, bd = 1 << 30;
    for (int g = 0; g < 1024; g++) {
      int dd = 0;
      uint32_t r = c;
      for (int j = 0; j < 8; j++, r /= 3) {
        const int a = kIq2sLevel[r % 3], v = (int)((m->iq2s[g] >> (8 * j)) & 0xff);
        dd += (a - v) * (a - v);
      }
      if (dd < bd) bd = dd, best = g;
    }
    m->near2[c] = (uint16_t)best;
  }
  return m;
}

// IQ3_XXS: per sub-block of 32 a step amax / 62 as d (2 s + 1) / 4, d = the largest step 4 / 31; each group of four
// magnitudes to the nearest levels, then to the nearest grid entry; in each sign group of eight the sign of the
// smallest magnitude flipped where needed to make the count of negatives even (the eighth sign is implied).
void quant_iq3_xxs(const float *x, uint8_t *y, uint32_t n) {
  const CodebookMaps &cb = *g_cb;
  for (uint32_t b = 0; b < n / 256; b++, x += 256, y += 98) {
    std::memset(y, 0, 98);
    float step[8];
    for (int j = 0; j < 8; j++) {
      float a = 0.0f;
      for (int i = 0; i < 32; i++) a = std::max(a, std::fabs(x[32 * j + i]));
      step[j] = a / 62.0f;
    }
    const float smax = *std::max_element(step, step + 8);
    const uint16_t dh = fp16_bits(smax * 4.0f / 31.0f);
    const float d = fp16_value(dh);
    std::memcpy(y, &dh, 2);
    if (d <= 0.0f) continue;
    for (int ib = 0; ib < 8; ib++) {
      const int s = std::clamp(nearest((step[ib] * 4.0f / d - 1.0f) / 2.0f), 0, 15);
      const float db = d * (float)(2 * s + 1) / 4.0f;
      uint32_t word = (uint32_t)s << 28;
      for (int l = 0; l < 4; l++) {
        const float *v = x + 32 * ib + 8 * l;
        uint32_t sb = 0;
        int small = 0;
        for (int j = 0; j < 8; j++) {
          if (v[j] < 0.0f) sb |= 1u << j;
          if (std::fabs(v[j]) < std::fabs(v[small])) small = j;
        }
        if (__builtin_popcount(sb) & 1) sb ^= 1u << small;
        word |= (sb & 127u) << (7 * l);
        for (int h = 0; h < 2; h++) {
          uint32_t code = 0;
          for (int j = 0; j < 4; j++)
            code |= (uint32_t)std::clamp(nearest((std::fabs(v[4 * h + j]) / db - 4.0f) / 8.0f), 0, 7) << (3 * j);
          y[2 + 8 * ib + 2 * l + h] = (uint8_t)cb.near3[code];
        }
      }
      std::memcpy(y + 66 + 4 * ib, &word, 4);
    }
  }
}

// IQ2_S: per half sub-block of 16 a step amax / 43 as d (2 s + 1) / 8, d = the largest step 8 / 31; each group of
// eight magnitudes to the nearest levels, then to the nearest grid entry; the signs stored plainly.
void quant_iq2_s(const float *x, uint8_t *y, uint32_t n) {
  const CodebookMaps &cb = *g_cb;
  for (uint32_t b = 0; b < n / 256; b++, x += 256, y += 82) {
    std::memset(y, 0, 82);
    float step[16];
    for (int h = 0; h < 16; h++) {
      float a = 0.0f;
      for (int i = 0; i < 16; i++) a = std::max(a, std::fabs(x[16 * h + i]));
      step[h] = a / 43.0f;
    }
    const float smax = *std::max_element(step, step + 16);
    const uint16_t dh = fp16_bits(smax * 8.0f / 31.0f);
    const float d = fp16_value(dh);
    std::memcpy(y, &dh, 2);
    if (d <= 0.0f) continue;
    for (int h = 0; h < 16; h++) {
      const int s = std::clamp(nearest((step[h] * 8.0f / d - 1.0f) / 2.0f), 0, 15);
      y[74 + h / 2] |= (uint8_t)(s << (4 * (h % 2)));
      const float db = d * (float)(2 * s + 1) / 8.0f;
      for (int g2 = 0; g2 < 2; g2++) {  // the half's two groups of eight: group g = 2 (h % 2) + g2 of sub-block h / 2
        const int ib = h / 2, g = 2 * (h % 2) + g2;
        const float *v = x + 32 * ib + 8 * g;
        uint32_t code = 0, mul = 1;
        uint8_t sb = 0;
        for (int j = 0; j < 8; j++, mul *= 3) {
          const float a = std::fabs(v[j]) / db;
          const int l = a < 16.5f ? 0 : a < 34.0f ? 1 : 2;
          code += (uint32_t)l * mul;
          if (v[j] < 0.0f) sb |= (uint8_t)(1u << j);
        }
        const uint32_t idx = cb.near2[code];
        y[2 + 4 * ib + g] = (uint8_t)(idx & 0xff);
        y[66 + ib] |= (uint8_t)(((idx >> 8) & 3u) << (2 * g));
        y[34 + 4 * ib + g] = sb;
      }
    }
  }
}

// IQ4_NL (block_iq4_nl): per block of 32 the value of largest magnitude m, d = m / -127 (kvalues_iq4nl's first
// entry), each value the nearest table entry of x / d. Simpler than ggml's scale search; any d and codes are a valid
// block, and the tests read the blocks the same way on both sides.
constexpr int8_t kIq4nl[16] = {-127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113};
void quant_iq4_nl(const float *x, uint8_t *y, uint32_t n) {
  for (uint32_t b = 0; b < n / 32; b++, x += 32, y += 18) {
    float m = 0.0f;
    for (int j = 0; j < 32; j++)
      if (std::fabs(x[j]) > std::fabs(m)) m = x[j];
    const uint16_t dh = fp16_bits(m / -127.0f);
    const float d = fp16_value(dh), id = d != 0.0f ? 1.0f / d : 0.0f;
    std::memcpy(y, &dh, 2);
    uint8_t code[32];
    for (int j = 0; j < 32; j++) {
      const float v = x[j] * id;
      int best = 0;
      for (int k = 1; k < 16; k++)
        if (std::fabs(v - kIq4nl[k]) < std::fabs(v - kIq4nl[best])) best = k;
      code[j] = (uint8_t)best;
    }
    for (int j = 0; j < 16; j++) y[2 + j] = (uint8_t)(code[j] | (code[j + 16] << 4));
  }
}

// Q2_0 (block_q2_0): per block of 64, d = amax / 2 and code q = clamp(round(x / d) + 1, 0, 3), y = (q - 1) d.
void quant_q2_0(const float *x, uint8_t *y, uint32_t n) {
  for (uint32_t b = 0; b < n / 64; b++, x += 64, y += 18) {
    float amax = 0.0f;
    for (int j = 0; j < 64; j++) amax = std::max(amax, std::fabs(x[j]));
    const uint16_t dh = fp16_bits(amax / 2.0f);
    const float d = fp16_value(dh), id = d != 0.0f ? 1.0f / d : 0.0f;
    std::memcpy(y, &dh, 2);
    std::memset(y + 2, 0, 16);
    for (int j = 0; j < 64; j++) {
      const int q = std::min(3, std::max(0, nearest(x[j] * id) + 1));
      y[2 + j / 4] |= (uint8_t)(q << (2 * (j % 4)));
    }
  }
}

// Q5_K: Q4_K's scheme with 31 steps a sub-block; the fifth bit of each code goes to qh (bit j of byte l for value
// 32 j + l). Valid blocks, not ggml's search.
void quant_q5_K(const float *x, uint8_t *y, uint32_t n) {
  for (uint32_t b = 0; b < n / 256; b++, x += 256, y += 176) {
    float step[8], mins[8];
    for (int j = 0; j < 8; j++) {
      float lo = 0.0f, hi = 0.0f;
      for (int i = 0; i < 32; i++) lo = std::min(lo, x[32 * j + i]), hi = std::max(hi, x[32 * j + i]);
      mins[j] = -lo;
      step[j] = (hi - lo) / 31.0f;
    }
    const float smax = *std::max_element(step, step + 8), mmax = *std::max_element(mins, mins + 8);
    const uint16_t dh = fp16_bits(smax / 63.0f), mh = fp16_bits(mmax / 63.0f);
    const float d = fp16_value(dh), dmin = fp16_value(mh);
    int sc[8], m[8];
    for (int j = 0; j < 8; j++) {
      sc[j] = d > 0.0f ? std::clamp(nearest(step[j] / d), 0, 63) : 0;
      m[j] = dmin > 0.0f ? std::clamp(nearest(mins[j] / dmin), 0, 63) : 0;
      if (step[j] > 0.0f && sc[j] == 0) sc[j] = 1;
    }
    std::memset(y, 0, 176);
    std::memcpy(y, &dh, 2);
    std::memcpy(y + 2, &mh, 2);
    uint8_t *s = y + 4;
    for (int j = 0; j < 4; j++) {
      s[j] = (uint8_t)((sc[j] & 63) | ((sc[j + 4] >> 4) << 6));
      s[j + 4] = (uint8_t)((m[j] & 63) | ((m[j + 4] >> 4) << 6));
      s[j + 8] = (uint8_t)((sc[j + 4] & 15) | ((m[j + 4] & 15) << 4));
    }
    uint8_t q[256];
    for (int j = 0; j < 8; j++) {
      const float dj = d * (float)sc[j], mj = dmin * (float)m[j];
      for (int i = 0; i < 32; i++) q[32 * j + i] = dj > 0.0f ? (uint8_t)std::clamp(nearest((x[32 * j + i] + mj) / dj), 0, 31) : 0;
    }
    uint8_t *qh = y + 16, *qs = y + 48;
    for (int v = 0; v < 256; v++) qh[v % 32] |= (uint8_t)(((q[v] >> 4) & 1) << (v / 32));
    for (int c = 0; c < 4; c++)
      for (int l = 0; l < 32; l++) qs[32 * c + l] = (uint8_t)((q[64 * c + l] & 15) | ((q[64 * c + 32 + l] & 15) << 4));
  }
}

// Q6_K: per sub-block of 16 a step amax / 31 as d sc, d = the largest step / 127 (signed scales: the sub-block's
// value of largest magnitude sets the sign, so that its code is -31); codes q - 32 = round(x / (d sc)), clamped.
void quant_q6_K(const float *x, uint8_t *y, uint32_t n) {
  for (uint32_t b = 0; b < n / 256; b++, x += 256, y += 210) {
    float st[16];
    for (int j = 0; j < 16; j++) {
      float m = 0.0f;
      for (int i = 0; i < 16; i++)
        if (std::fabs(x[16 * j + i]) > std::fabs(m)) m = x[16 * j + i];
      st[j] = m / -31.0f;
    }
    float amax = 0.0f;
    for (int j = 0; j < 16; j++) amax = std::max(amax, std::fabs(st[j]));
    const uint16_t dh = fp16_bits(amax / 127.0f);
    const float d = fp16_value(dh);
    std::memset(y, 0, 210);
    int8_t *sc = (int8_t *)(y + 192);
    uint8_t q[256];
    for (int j = 0; j < 16; j++) {
      sc[j] = (int8_t)(d > 0.0f ? std::clamp(nearest(st[j] / d), -127, 127) : 0);
      const float dj = d * (float)sc[j];
      for (int i = 0; i < 16; i++)
        q[16 * j + i] = (uint8_t)(dj != 0.0f ? std::clamp(nearest(x[16 * j + i] / dj), -32, 31) + 32 : 32);
    }
    uint8_t *ql = y, *qh = y + 128;
    for (int v = 0; v < 256; v++) {  // v = 128 h + 32 j + l
      const int h = v / 128, j = (v % 128) / 32, l = v % 32;
      ql[64 * h + 32 * (j % 2) + l] |= (uint8_t)((q[v] & 15) << (4 * (j / 2)));
      qh[32 * h + l] |= (uint8_t)((q[v] >> 4) << (2 * j));
    }
    std::memcpy(y + 208, &dh, 2);
  }
}

// IQ4_XS: per sub-block of 32 a step (the value of largest magnitude / -127, kvalues' first entry) as d (ls - 32),
// d = the largest step's magnitude / 32 with the sign that lets ls - 32 reach -32; codes the nearest table entries.
void quant_iq4_xs(const float *x, uint8_t *y, uint32_t n) {
  for (uint32_t b = 0; b < n / 256; b++, x += 256, y += 136) {
    float st[8], amax = 0.0f;
    for (int j = 0; j < 8; j++) {
      float m = 0.0f;
      for (int i = 0; i < 32; i++)
        if (std::fabs(x[32 * j + i]) > std::fabs(m)) m = x[32 * j + i];
      st[j] = m / -127.0f;
      amax = std::max(amax, std::fabs(st[j]));
    }
    const uint16_t dh = fp16_bits(-amax / 32.0f);
    const float d = fp16_value(dh);
    std::memset(y, 0, 136);
    std::memcpy(y, &dh, 2);
    uint16_t sh = 0;
    for (int j = 0; j < 8; j++) {
      const int ls = d != 0.0f ? std::clamp(nearest(st[j] / d), -32, 31) + 32 : 32;
      y[4 + j / 2] |= (uint8_t)((ls & 15) << (4 * (j % 2)));
      sh |= (uint16_t)(((ls >> 4) & 3) << (2 * j));
      const float dl = d * (float)(ls - 32), id = dl != 0.0f ? 1.0f / dl : 0.0f;
      uint8_t code[32];
      for (int i = 0; i < 32; i++) {
        const float v = x[32 * j + i] * id;
        int best = 0;
        for (int k = 1; k < 16; k++)
          if (std::fabs(v - kIq4nl[k]) < std::fabs(v - kIq4nl[best])) best = k;
        code[i] = (uint8_t)best;
      }
      for (int i = 0; i < 16; i++) y[8 + 16 * j + i] = (uint8_t)(code[i] | (code[i + 16] << 4));
    }
    std::memcpy(y + 2, &sh, 2);
  }
}

// Whether a row of cols values is whole blocks of a GPU type (and, for the codebook types, the codebooks are set).
bool cols_ok(uint32_t type, uint32_t cols) {
  const uint32_t bv = quant_block_values(type);
  if (quant_needs_codebook(type)) {
    std::lock_guard<std::mutex> g(g_cb_mu);
    if (!g_cb) return false;
  }
  return quant_gpu_supported(type) && bv && cols % bv == 0 && cols > 0;
}

bool quant_rows(uint32_t type, const float *x, uint32_t cols, uint8_t *out) {
  switch (type) {
    case QT_Q8_0: quant_q8_0(x, out, cols); return true;
    case QT_Q4_K: quant_q4_K(x, out, cols); return true;
    case QT_IQ3_S: quant_iq3_s(x, out, cols); return true;
    case QT_IQ4_NL: quant_iq4_nl(x, out, cols); return true;
    case QT_Q2_0: quant_q2_0(x, out, cols); return true;
    case QT_IQ3_XXS: quant_iq3_xxs(x, out, cols); return true;
    case QT_IQ2_S: quant_iq2_s(x, out, cols); return true;
    case QT_Q5_K: quant_q5_K(x, out, cols); return true;
    case QT_Q6_K: quant_q6_K(x, out, cols); return true;
    case QT_IQ4_XS: quant_iq4_xs(x, out, cols); return true;
    default: return false;
  }
}

}  // namespace
}  // namespace c0ven

using namespace c0ven;

extern "C" {

MOE_API uint64_t moe_row_bytes(uint32_t type, uint32_t cols) {
  const uint32_t bv = quant_block_values(type);
  return bv ? (uint64_t)cols / bv * quant_block_bytes(type) : 0;
}

MOE_API moe_status moe_synth_set_codebooks(const uint8_t *qgrid, uint64_t bytes) {
  if (!qgrid || bytes < QGRID_IQ3S) return MOE_BAD_ARGUMENT;
  CodebookMaps *m = make_maps(qgrid);
  std::lock_guard<std::mutex> g(g_cb_mu);
  g_cb = m;  // an earlier set stays allocated: a quantiser running on another thread may still read it
  return MOE_OK;
}

MOE_API void moe_synth_normal(uint64_t seed, uint64_t stream, float sigma, float *out, uint64_t n, int nthreads) {
  const Normal nr(seed, stream);
  const uint64_t chunk = 1 << 16, nc = (n + chunk - 1) / chunk;
  parallel_for(nc, nthreads, [&](uint64_t c) {
    const uint64_t i0 = c * chunk;
    nr.fill(sigma, out + i0, i0, std::min(chunk, n - i0));
  });
}

MOE_API moe_status moe_quantize(uint32_t type, const float *x, uint32_t rows, uint32_t cols, uint8_t *out,
                                int nthreads) {
  if (!cols_ok(type, cols)) return MOE_BAD_ARGUMENT;
  const uint64_t rb = moe_row_bytes(type, cols);
  parallel_for(rows, nthreads, [&](uint64_t r) { quant_rows(type, x + r * cols, cols, out + r * rb); });
  return MOE_OK;
}

MOE_API moe_status moe_synth_matrix(uint64_t seed, uint64_t stream, float sigma, uint32_t type, uint32_t rows,
                                    uint32_t cols, uint8_t *out, int nthreads) {
  if (!cols_ok(type, cols)) return MOE_BAD_ARGUMENT;
  const Normal nr(seed, stream);
  const uint64_t rb = moe_row_bytes(type, cols);
  const uint64_t per = std::max<uint64_t>(1, (1u << 16) / cols), nc = (rows + per - 1) / per;
  parallel_for(nc, nthreads, [&](uint64_t c) {
    std::vector<float> buf((size_t)per * cols);
    const uint64_t r0 = c * per, nr_ = std::min<uint64_t>(per, rows - r0);
    nr.fill(sigma, buf.data(), r0 * cols, nr_ * cols);
    for (uint64_t r = 0; r < nr_; r++) quant_rows(type, buf.data() + r * cols, cols, out + (r0 + r) * rb);
  });
  return MOE_OK;
}

MOE_API void moe_zipf_bias(uint64_t seed, uint32_t n_expert, float s, float *out) {
  std::vector<uint32_t> perm(n_expert);
  for (uint32_t i = 0; i < n_expert; i++) perm[i] = i;
  uint64_t st = splitmix64(seed ^ 0x5a17f00dull);
  for (uint32_t i = n_expert; i > 1; i--) {  // Fisher-Yates
    st = splitmix64(st);
    std::swap(perm[i - 1], perm[st % i]);
  }
  for (uint32_t e = 0; e < n_expert; e++) out[e] = (float)(-(double)s * std::log(1.0 + (double)perm[e]));
}

}  // extern "C"
