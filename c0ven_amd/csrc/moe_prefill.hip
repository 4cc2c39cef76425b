// The prefill path of the MoE block: router GEMM, top-k, counting-sort dispatch, grouped int8-MFMA expert GEMMs and
// the combine. The kernel list and its reference counterparts are in prefill.h.
//
// Bits: every result equals the CPU oracle's (its ORACLE ORDER). The router sums exact bf16 products in fp64 in k
// order, as the oracle does. The expert GEMMs (pf_gemm16) take exact int32 block or unit sums from 16 x 16 int8 MFMA
// tiles (mfma_q4k.h, mfma_iq3s.h, mfma_q8_0.h), then follow each unit's fp32 steps exactly as the decoders in units.h
// do, and add a row's units in sequence, as the oracle does.
#include <hip/hip_runtime.h>

#include <type_traits>

#include "act_quant.h"
#include "device_math.h"
#include "iq3s_grid.h"
#include "layout.h"
#include "mfma_iq3s.h"
#include "mfma_kq.h"
#include "mfma_q4k.h"
#include "mfma_q8_0.h"
#include "prefill.h"
#include "route.h"

namespace c0ven {

constexpr uint32_t kMaxRouteExperts = 512;  // routed experts a layer may have

__device__ __constant__ static const uint32_t kIq3sGridPf[512] = {C0VEN_IQ3S_GRID_VALUES};

namespace {

constexpr uint32_t kPfWG = 256;

// The thread index, read afresh where it is used (the empty asm hides that it is the same value everywhere), so the
// compiler recomputes what derives from it at the use instead of hoisting it out of the loops and spilling it.
__device__ __forceinline__ uint32_t tid_fresh() {
  uint32_t t = threadIdx.x;
  asm volatile("" : "+v"(t));
  return t;
}
__device__ __forceinline__ uint32_t lane_id() { return tid_fresh() & 63u; }
__device__ __forceinline__ uint32_t wave_id() { return tid_fresh() >> 6; }

// ---------------------------------------------------------------------------------------------------------------
// Activation units: one half-wave per (row, unit), eight values a lane; o2 (a second type) may be null. The codes are
// stored in the matrix-core order (mfma_code_off), which every prefill GEMM reads.

// The quantiser's exchanges inside 16-lane rows as DPP moves (routed h at config 4: 14.2 -> 13.7 us).
constexpr bool kQuantDpp = true;

__global__ void __launch_bounds__(kPfWG) pf_quant_rows(const float *src, uint64_t ld, uint32_t rows, uint32_t U,
                                                       uint32_t t1, uint8_t *o1, uint32_t t2, uint8_t *o2) {
  const uint32_t hw = blockIdx.x * (kPfWG / 32) + threadIdx.x / 32, l32 = threadIdx.x & 31u;
  const uint32_t row = hw / U, u = hw % U;
  if (row >= rows) return;  // whole half-waves leave together
  // A row has ld values: past them (a partial last unit) the values are zeros (their q8_0 blocks: d 0, codes 0).
  const uint32_t v0 = u * kUnit + 8 * l32;
  float4 a = make_float4(0.0f, 0.0f, 0.0f, 0.0f), b = a;
  if (v0 < ld) {
    const float4 *p = (const float4 *)(src + (uint64_t)row * ld + v0);
    a = p[0], b = p[1];
  }
  const float v[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
  quant_unit<false, true, true, true, kQuantDpp>(v, l32, t1, o1 + ((uint64_t)row * U + u) * kActBytes);
  if (o2) quant_unit<false, true, true, true, kQuantDpp>(v, l32, t2, o2 + ((uint64_t)row * U + u) * kActBytes);
}

// Work-group b (< n) of a 1-D grid runs on XCD b % 8 (the dispatcher deals work-groups to the eight XCDs in turn), as
// the (b / 8)-th of the cnt_x = floor((n - x + 7) / 8) that XCD x receives among the first n. Its logical index puts
// consecutive logical indices on one XCD: XCD x takes [off_x, off_x + cnt_x), off_x = x floor(n / 8) + min(x, n % 8),
// a bijection of [0, n) for any n. With the row block fastest in the logical index, a tile's row blocks run together
// on one XCD (its activations come from that XCD's L2), and the next tile of the same expert follows on the same XCD
// (its weights too). The caller returns for b >= n.
__device__ __forceinline__ uint32_t xcd_logical(uint32_t b, uint32_t n) {
  const uint32_t x = b % 8, q = n / 8, r = n % 8;
  return x * q + min(x, r) + b / 8;
}

// h = silu(g) u of gate and up rows computed apart (a shared expert whose gate and up differ in type), quantised as
// pf_quant_rows quantises h: the same SwiGLU as the fused gate/up kernels' epilogue, then the same units.
__global__ void __launch_bounds__(kPfWG) pf_quant_swiglu(const float *g, const float *up, uint32_t ld, uint32_t rows,
                                                         uint32_t U, float limit, uint32_t t1, uint8_t *o1) {
  __shared__ uint64_t tab[32];
  if (threadIdx.x < 32) tab[threadIdx.x] = kExp2Tab[threadIdx.x];
  __syncthreads();
  const uint32_t hw = blockIdx.x * (kPfWG / 32) + threadIdx.x / 32, l32 = threadIdx.x & 31u;
  const uint32_t row = hw / U, u = hw % U;
  if (row >= rows) return;
  const uint32_t v0 = u * kUnit + 8 * l32;
  float v[8] = {0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f};
  if (v0 < ld) {
    const float4 *pg = (const float4 *)(g + (uint64_t)row * ld + v0), *pu = (const float4 *)(up + (uint64_t)row * ld + v0);
    const float4 g0 = pg[0], g1 = pg[1], u0 = pu[0], u1 = pu[1];
    const float gv[8] = {g0.x, g0.y, g0.z, g0.w, g1.x, g1.y, g1.z, g1.w};
    const float uv[8] = {u0.x, u0.y, u0.z, u0.w, u1.x, u1.y, u1.z, u1.w};
#pragma unroll
    for (int i = 0; i < 8; i++) v[i] = swiglu_one(gv[i], uv[i], limit, tab);
  }
  quant_unit<false, true, true, true, kQuantDpp>(v, l32, t1, o1 + ((uint64_t)row * U + u) * kActBytes);
}

// ---------------------------------------------------------------------------------------------------------------
// Router: a 64-token x 64-row tile per work-group (rows < E) on the fp64 matrix cores. v_mfma_f64_16x16x4_f64 adds its
// four k terms to the accumulator one fused multiply-add after another in k order (checked against the fma chain), so
// a chain of them over k = 0, 4, 8, ... is the oracle's sum term for term. Wave w takes rows 32 (w % 2) .. and tokens
// 32 (w / 2) .. as 2 x 2 tiles of 16 x 16. K goes in chunks of 32 staged as doubles in two LDS buffers: chunk c + 1 is
// loaded into registers while chunk c is used, and stored to the other buffer after it (one barrier a chunk). The
// shared gate's row E takes an extra row of work-groups: a thread a token, k ascending; they also clear their 64-token
// window's dispatch masks for pf_topk.
// logits[t][e] = (float)(sum over k ascending of bf16(W[e][k]) bf16(x[t][k]), each product exact, in fp64)
// (+ bias[e] for e < E).

constexpr uint32_t kRtK = 32, kRtPad = 66;  // the padded row of a staged k (doubles): the four k of a step fall apart

typedef double v4d_t __attribute__((ext_vector_type(4)));

__global__ void __launch_bounds__(kPfWG) pf_router(const float *x, uint32_t T, const uint16_t *W, const float *bias,
                                                   uint32_t E, uint32_t H, float *logits, unsigned long long *masks) {
  __shared__ double xs[2][kRtK][kRtPad], ws[2][kRtK][kRtPad];
  const uint32_t t0 = blockIdx.x * 64, e0 = blockIdx.y * 64, tid = threadIdx.x;
  if (e0 >= E) {  // the gate row: thread t of the first 64 a token
    for (uint32_t i = tid; i < E; i += kPfWG) masks[(uint64_t)blockIdx.x * E + i] = 0ull;  // the window's masks
    double *wrow = &ws[0][0][0];  // W[E] as doubles, 2048 a pass
    const uint32_t t = t0 + tid;
    double acc = 0.0;
    for (uint32_t k0 = 0; k0 < H; k0 += 2048) {
      const uint32_t nk = min(2048u, H - k0);
      __syncthreads();
      for (uint32_t k = tid; k < nk; k += kPfWG) wrow[k] = (double)bf2f(W[(uint64_t)E * H + k0 + k]);
      __syncthreads();
      if (tid < 64 && t < T) {
        const float4 *xr = (const float4 *)(x + (uint64_t)t * H + k0);
        for (uint32_t k = 0; k < nk; k += 32) {
          float4 q[8];
#pragma unroll
          for (int i = 0; i < 8; i++) q[i] = xr[k / 4 + i];
#pragma unroll
          for (int i = 0; i < 8; i++) {
            acc = __builtin_fma(wrow[k + 4 * i], (double)round_bf16(q[i].x), acc);
            acc = __builtin_fma(wrow[k + 4 * i + 1], (double)round_bf16(q[i].y), acc);
            acc = __builtin_fma(wrow[k + 4 * i + 2], (double)round_bf16(q[i].z), acc);
            acc = __builtin_fma(wrow[k + 4 * i + 3], (double)round_bf16(q[i].w), acc);
          }
        }
      }
    }
    if (tid < 64 && t < T) logits[(uint64_t)t * (E + 1) + E] = (float)acc;
    return;
  }
  const uint32_t l = lane_id(), w = wave_id(), g = l / 16, c16 = l % 16;
  const uint32_t rb = 32 * (w % 2), tb = 32 * (w / 2);  // the wave's rows and tokens within the tile
  const uint32_t sr = tid / 4, sk = 8 * (tid % 4);      // staging: row / token sr, values sk .. sk + 7
  v4d_t acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; i++)
#pragma unroll
    for (int j = 0; j < 2; j++) acc[i][j] = v4d_t{0.0, 0.0, 0.0, 0.0};
  float xv[8];
  uint4 wv;
  auto fetch = [&](uint32_t k0) {
    if (t0 + sr < T) {
      const float4 *p = (const float4 *)(x + (uint64_t)(t0 + sr) * H + k0 + sk);
      const float4 a = p[0], b = p[1];
      xv[0] = a.x, xv[1] = a.y, xv[2] = a.z, xv[3] = a.w, xv[4] = b.x, xv[5] = b.y, xv[6] = b.z, xv[7] = b.w;
    } else {
#pragma unroll
      for (int i = 0; i < 8; i++) xv[i] = 0.0f;
    }
    wv = e0 + sr < E ? *(const uint4 *)(W + (uint64_t)(e0 + sr) * H + k0 + sk) : make_uint4(0, 0, 0, 0);
  };
  auto stage = [&](uint32_t buf) {
    const uint32_t ww[4] = {wv.x, wv.y, wv.z, wv.w};
#pragma unroll
    for (int i = 0; i < 8; i++) {
      xs[buf][sk + i][sr] = (double)round_bf16(xv[i]);
      ws[buf][sk + i][sr] = (double)__uint_as_float((i & 1) ? ww[i / 2] & 0xffff0000u : ww[i / 2] << 16);
    }
  };
  fetch(0);
  stage(0);
  __syncthreads();
  for (uint32_t k0 = 0, c = 0; k0 < H; k0 += kRtK, c ^= 1u) {
    const bool more = k0 + kRtK < H;
    if (more) fetch(k0 + kRtK);
#pragma unroll
    for (uint32_t s = 0; s < kRtK / 4; s++) {
      const uint32_t k = 4 * s + g;
      const double a0 = ws[c][k][rb + c16], a1 = ws[c][k][rb + 16 + c16];
      const double b0 = xs[c][k][tb + c16], b1 = xs[c][k][tb + 16 + c16];
      acc[0][0] = __builtin_amdgcn_mfma_f64_16x16x4f64(a0, b0, acc[0][0], 0, 0, 0);
      acc[0][1] = __builtin_amdgcn_mfma_f64_16x16x4f64(a0, b1, acc[0][1], 0, 0, 0);
      acc[1][0] = __builtin_amdgcn_mfma_f64_16x16x4f64(a1, b0, acc[1][0], 0, 0, 0);
      acc[1][1] = __builtin_amdgcn_mfma_f64_16x16x4f64(a1, b1, acc[1][1], 0, 0, 0);
    }
    if (more) stage(c ^ 1u);
    __syncthreads();
  }
  // acc[i][j][q]: row rb + 16 i + g + 4 q, token tb + 16 j + c16.
#pragma unroll
  for (int i = 0; i < 2; i++)
#pragma unroll
    for (int j = 0; j < 2; j++)
#pragma unroll
      for (int q = 0; q < 4; q++) {
        const uint32_t t = t0 + tb + 16 * j + c16, e = e0 + rb + 16 * i + g + 4 * q;
        if (t < T && e < E) {
          float lg = (float)acc[i][j][q];
          if (bias) lg = __fadd_rn(lg, bias[e]);
          logits[(uint64_t)t * (E + 1) + e] = lg;
        }
      }
}

// ---------------------------------------------------------------------------------------------------------------
// Top-k: one wave a token (the decode kernel's steps, route.h, in one wave); each chosen expert's bit goes into the
// token's window mask for the dispatch.

__global__ void __launch_bounds__(kPfWG) pf_topk(const float *logits, uint32_t T, uint32_t E, uint32_t K,
                                                 int32_t *ids, float *w, float *gs, unsigned long long *masks) {
  __shared__ uint64_t tab[32];
  if (threadIdx.x < 32) tab[threadIdx.x] = kExp2Tab[threadIdx.x];
  __syncthreads();
  const uint32_t t = blockIdx.x * (kPfWG / 64) + wave_id(), lane = lane_id();
  if (t >= T) return;
  const float *lg = logits + (uint64_t)t * (E + 1);
  uint32_t key[kRoutePer], id[kRoutePer], my_id, my_key;
  route_load<false>(lg, E, lane, key, id);
  float mx, inv;
  route_norm(key, E, lane, tab, &mx, &inv);
  route_select(key, id, K, lane, &my_id, &my_key);
  const float wk = route_weight(my_key, mx, inv, K, lane, tab);
  if (lane < K) {
    ids[(uint64_t)t * K + lane] = (int32_t)my_id;
    w[(uint64_t)t * K + lane] = wk;
    atomicOr(&masks[(uint64_t)(t / 64) * E + my_id], 1ull << (t % 64));  // the dispatch's window mask
  }
  if (lane == 0 && gs) gs[t] = sigmoid_libm(lg[E], tab);
}

// ---------------------------------------------------------------------------------------------------------------
// The router on the bf16 matrix cores, with certified top-k. The logits come from v_mfma_f32_16x16x32_bf16 (every
// bf16 x bf16 product exact, sums in fp32) instead of the fp64 k-order sum; each is within a bound of the exact one,
// and where the bound leaves the top k or their order open, the experts that could be among them are summed again
// exactly before the selection. So ids are the oracle's; the weights and the shared gate are computed from logits
// within ~1e-6 of the oracle's (the block output within its tolerance, not bit for bit).
//
// The bound. A work-group takes 32 rows x 32 tokens; its four waves take a quarter of K each. Every MFMA starts from
// zero (32 products, at most 31 roundings inside), its result is added to the wave's fp32 sum (one rounding a chunk),
// and the four quarters are added in order (three more): at most n = 31 + H / 128 + 3 roundings touch any product,
// each of relative size at most 2^-23 whatever the rounding mode, so |l~ - l| <= 1.01 n 2^-23 sum_k |w_k x_k| <=
// gamma ||W_e|| ||bf16(x_t)|| (Cauchy-Schwarz); rounding the sum to fp32 and adding the bias add at most
// 2^-23 (|l~| + |bias|) more.
//
// The exact sums. Every product w x of two bf16 values is a multiple of 2^(lsb(w) + lsb(x)) (lsb: the weight of the
// value's last mantissa bit), and so is every partial sum of the row's products. When sum_k |w_k x_k| < 2^(L + 53),
// L = min_k lsb(W_e[k]) + min_k lsb(x_t[k]), every partial sum, in any order, is exact in fp64: the oracle's k-order
// double sum is that exact value, and so is a parallel sum. Then eight lanes sum an expert's row (a contiguous eighth
// each, then a fixed tree); otherwise one lane runs the k-order chain.

// The weight of a bf16 value's last mantissa bit as a power of two (normal: exponent - 7; subnormal: -133); zero
// contributes nothing (a large sentinel).
__device__ __forceinline__ int bf16_lsb(uint32_t b) {
  const uint32_t ex = (b >> 7) & 0xffu;
  return (b & 0x7fffu) == 0 ? 1 << 20 : ex == 0 ? -133 : (int)ex - 134;
}

// x to bf16 (round to nearest even), its norm ||bf16(x_t)||_2 rounded up and the least lsb of its values; the dispatch
// masks cleared. One wave a token.
// bf16 operands of the router's matrix-core products in tiles of 16 rows x 32 values (1 KB, the 32 values of a row
// contiguous), tile (row / 16, k / 32) at ((row / 16) (H / 32) + k / 32) 512 elements: a wave's operand load of one
// tile reads its 1 KB whole, and a row block's K walk is one contiguous run.
__device__ __forceinline__ uint64_t tile16x32(uint32_t row, uint32_t k, uint32_t H) {
  return ((uint64_t)(row / 16) * (H / 32) + k / 32) * 512 + (row % 16) * 32 + k % 32;
}

__global__ void __launch_bounds__(kPfWG) pf_xprep(const float *x, uint32_t T, uint32_t H, uint32_t E, uint16_t *xb,
                                                  uint16_t *xt, float *xn, int *xlsb, unsigned long long *masks,
                                                  const uint16_t *wg, float *logits, float *gs) {
  __shared__ uint64_t tab[32];
  if (threadIdx.x < 32) tab[threadIdx.x] = kExp2Tab[threadIdx.x];
  __syncthreads();
  const uint32_t t = blockIdx.x * (kPfWG / 64) + wave_id(), lane = lane_id();
  for (uint32_t i = blockIdx.x * kPfWG + threadIdx.x; i < pf_windows(T) * E; i += gridDim.x * kPfWG) masks[i] = 0ull;
  if (t >= T) return;
  double ss = 0.0;
  int lsb = 1 << 20;
  double gpart = 0.0;  // the shared gate's row against bf16(x): exact products, fp64 partials a lane
  // x's loads four chunks at a time, all issued before the first is used (one wave a token leaves few waves a CU, so
  // each dependent round trip would cost the whole latency).
  constexpr uint32_t kBatch = 4;
  for (uint32_t k0 = 8 * lane; k0 < H; k0 += 512 * kBatch) {
    float4 xa[kBatch], xb4[kBatch];
    uint4 wa[kBatch];
#pragma unroll
    for (uint32_t j = 0; j < kBatch; j++) {
      const uint32_t k = k0 + 512 * j < H ? k0 + 512 * j : k0;
      const float4 *p = (const float4 *)(x + (uint64_t)t * H + k);
      xa[j] = p[0], xb4[j] = p[1];
      if (gs) wa[j] = *(const uint4 *)(wg + k);
    }
#pragma unroll
    for (uint32_t j = 0; j < kBatch; j++) {
      const uint32_t k = k0 + 512 * j;
      if (k >= H) break;
      const float4 a = xa[j], b = xb4[j];
      const float v[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
      uint32_t o[4];
#pragma unroll
      for (int i = 0; i < 4; i++) {
        float r0, r1;
        round_bf16_2(v[2 * i], v[2 * i + 1], r0, r1);
        ss = __builtin_fma((double)r0, (double)r0, ss);
        ss = __builtin_fma((double)r1, (double)r1, ss);
        o[i] = (__float_as_uint(r0) >> 16) | (__float_as_uint(r1) & 0xffff0000u);
        lsb = min(lsb, min(bf16_lsb(o[i] & 0xffffu), bf16_lsb(o[i] >> 16)));
      }
      if (gs) {
        const uint32_t aw[4] = {wa[j].x, wa[j].y, wa[j].z, wa[j].w};
#pragma unroll
        for (int i = 0; i < 4; i++) {
          gpart = __builtin_fma((double)__uint_as_float(aw[i] << 16), (double)__uint_as_float(o[i] << 16), gpart);
          gpart = __builtin_fma((double)__uint_as_float(aw[i] & 0xffff0000u),
                                (double)__uint_as_float(o[i] & 0xffff0000u), gpart);
        }
      }
      *(uint4 *)(xb + (uint64_t)t * H + k) = make_uint4(o[0], o[1], o[2], o[3]);
      *(uint4 *)(xt + tile16x32(t, k, H)) = make_uint4(o[0], o[1], o[2], o[3]);
    }
  }
  const double tot = wave_sum_f64(ss);
  lsb = -(int)wave_max_u32((uint32_t)(-lsb + (1 << 21))) + (1 << 21);
  const float le = gs ? (float)wave_sum_f64(gpart) : 0.0f;
  if (lane == 0) {
    xn[t] = (float)(sqrt(tot) * (1.0 + 0x1p-40)) * (1.0f + 0x1p-22f);
    xlsb[t] = lsb;
    if (gs) {  // the shared gate's logit (fp64 partials in another order than the oracle's chain: within the tolerance)
      logits[(uint64_t)t * (E + 1) + E] = le;
      gs[t] = sigmoid_libm(le, tab);
    }
  }
}

typedef __bf16 v8bf_t __attribute__((ext_vector_type(8)));
typedef float v4f_t __attribute__((ext_vector_type(4)));

// Approximate logits of rows < E: a 16 kS-row x 16 kS-token tile a work-group (1-D grid, XCD-aware: a token block's
// row blocks run on one XCD, so its bf16 x is fetched into that XCD's L2 once), wave w summing K range [w H / 4,
// (w + 1) H / 4). Operands straight from memory (the router's bf16 rows and the prepared bf16 x), kPre steps ahead.
// kS = 2: 64 x 64 tiles (kS = 4, one work-group a CU, half the bytes into each CU) measured 30 against 26 us.
constexpr uint32_t kRtPre = 4;  // steps of loads in flight; a wave's K steps (H / 128) are a multiple of it
template <uint32_t kS>
__global__ void __launch_bounds__(kPfWG) pf_router_bf16(const uint16_t *Wt, const uint16_t *xt, uint32_t T, uint32_t E,
                                                        uint32_t H, const float *bias, float *logits) {
  constexpr uint32_t kTile = 16 * kS;
  __shared__ v4f_t part[3][kS * kS][64];
  const uint32_t nrb = (E + kTile - 1) / kTile, ntb = (T + kTile - 1) / kTile, n = nrb * ntb;
  if (blockIdx.x >= n) return;
  const uint32_t L = xcd_logical(blockIdx.x, n), e0 = kTile * (L % nrb), t0 = kTile * (L / nrb);
  const uint32_t l = lane_id(), w = wave_id(), g = l / 16, c16 = l % 16;
  const uint32_t kq = H / 4, k0 = w * kq, ns = kq / 32;
  // Tiles past E rows or T tokens (the last 16-row tile's rows past them are whatever the buffers hold) read tile 0;
  // their results are never stored. A step advances one tile: 512 elements.
  const uint32_t lo = c16 * 32 + 8 * g;  // the lane's 8 values in a tile
  const uint16_t *pr[kS], *pt[kS];
#pragma unroll
  for (uint32_t i = 0; i < kS; i++) {
    const uint32_t r = e0 + 16 * i < E ? e0 + 16 * i : 0u, t = t0 + 16 * i < T ? t0 + 16 * i : 0u;
    pr[i] = Wt + tile16x32(r, k0, H) + lo, pt[i] = xt + tile16x32(t, k0, H) + lo;
  }
  v4f_t acc[kS][kS];
#pragma unroll
  for (uint32_t i = 0; i < kS; i++)
#pragma unroll
    for (uint32_t j = 0; j < kS; j++) acc[i][j] = v4f_t{0.0f, 0.0f, 0.0f, 0.0f};
  v8bf_t op[kRtPre][2 * kS];  // rows 0 .. kS - 1, then tokens
#pragma unroll
  for (uint32_t d = 0; d < kRtPre; d++) {
    const uint32_t k = 512 * min(d, ns - 1);
#pragma unroll
    for (uint32_t i = 0; i < kS; i++) op[d][i] = *(const v8bf_t *)(pr[i] + k), op[d][kS + i] = *(const v8bf_t *)(pt[i] + k);
  }
  // No branch inside the unrolled steps: the compiler's waits then count the loads in flight (a branch made it wait for
  // all of them, the prefetch lost). Each product tile's chain starts from zero and is added to the fp32 total.
  for (uint32_t s0 = 0; s0 < ns; s0 += kRtPre) {
#pragma unroll
    for (uint32_t d = 0; d < kRtPre; d++) {
      v4f_t dv[kS][kS];
#pragma unroll
      for (uint32_t i = 0; i < kS; i++)
#pragma unroll
        for (uint32_t j = 0; j < kS; j++)
          dv[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(op[d][i], op[d][kS + j], v4f_t{0.0f, 0.0f, 0.0f, 0.0f}, 0, 0, 0);
      const uint32_t kn = 512 * min(s0 + d + kRtPre, ns - 1);  // the load kPre steps ahead (the last again past the end)
#pragma unroll
      for (uint32_t i = 0; i < kS; i++)
        op[d][i] = *(const v8bf_t *)(pr[i] + kn), op[d][kS + i] = *(const v8bf_t *)(pt[i] + kn);
#pragma unroll
      for (uint32_t i = 0; i < kS; i++)
#pragma unroll
        for (uint32_t j = 0; j < kS; j++)
#pragma unroll
          for (int q = 0; q < 4; q++) acc[i][j][q] = __fadd_rn(acc[i][j][q], dv[i][j][q]);
    }
  }
  if (w > 0) {
#pragma unroll
    for (uint32_t i = 0; i < kS; i++)
#pragma unroll
      for (uint32_t j = 0; j < kS; j++) part[w - 1][kS * i + j][l] = acc[i][j];
  }
  __syncthreads();
  if (w != 0) return;
  // acc[i][j][q]: row e0 + 16 i + 4 g + q, token t0 + 16 j + c16.
#pragma unroll
  for (uint32_t i = 0; i < kS; i++)
#pragma unroll
    for (uint32_t j = 0; j < kS; j++) {
      v4f_t s = acc[i][j];
#pragma unroll
      for (int v = 0; v < 3; v++) {
        const v4f_t o = part[v][kS * i + j][l];
#pragma unroll
        for (int q = 0; q < 4; q++) s[q] = __fadd_rn(s[q], o[q]);
      }
#pragma unroll
      for (int q = 0; q < 4; q++) {
        const uint32_t t = t0 + 16 * j + c16, e = e0 + 16 * i + 4 * g + q;
        if (t < T && e < E) logits[(uint64_t)t * (E + 1) + e] = bias ? __fadd_rn(s[q], bias[e]) : s[q];
      }
    }
}

// Row e's exact logit for token t by the k-order chain: sum over k ascending of bf16(W[e][k]) bf16(x[t][k]) in fp64
// (each product exact, one fused step a term: the oracle's arithmetic), rounded to fp32. One lane.
__device__ __forceinline__ float exact_logit_chain(const uint16_t *W, const uint16_t *xb, uint32_t H, uint32_t e,
                                                   uint32_t t) {
  const uint4 *wr = (const uint4 *)(W + (uint64_t)e * H), *xr = (const uint4 *)(xb + (uint64_t)t * H);
  double acc = 0.0;
  for (uint32_t k = 0; k < H / 8; k++) {
    const uint4 a = wr[k], b = xr[k];
    const uint32_t aw[4] = {a.x, a.y, a.z, a.w}, bw[4] = {b.x, b.y, b.z, b.w};
#pragma unroll
    for (int i = 0; i < 4; i++) {
      acc = __builtin_fma((double)__uint_as_float(aw[i] << 16), (double)__uint_as_float(bw[i] << 16), acc);
      acc = __builtin_fma((double)__uint_as_float(aw[i] & 0xffff0000u), (double)__uint_as_float(bw[i] & 0xffff0000u), acc);
    }
  }
  return (float)acc;
}

// Top-k on the approximate logits, certified: with B the token's bound, the K winners and their order stand when each
// of the K + 1 largest keys exceeds the next by more than 2 B. Otherwise only the experts whose place is open are
// summed again exactly (sixteen lanes an expert, or one lane's k-order chain where the exactness condition fails):
// a ranked expert whose interval meets a neighbour's, and, when the K-th place is open, every later expert whose
// approximate logit reaches the K-th's - 2 B. The selection then runs again on the mixed keys. cnt_exact counts the
// tokens that needed exact sums. (The shared gate's logit and gs come from pf_xprep.)
__global__ void __launch_bounds__(kPfWG) pf_topk_cert(float *logits, const uint16_t *W, const int *rlsb,
                                                      const uint16_t *xb, const float *xn, const int *xlsb, uint32_t T,
                                                      uint32_t E, uint32_t H, uint32_t K, const float *bias,
                                                      float gamma_rmax, float bias_max, int32_t *ids, float *w,
                                                      unsigned long long *masks, uint32_t *cnt_exact) {
  __shared__ uint64_t tab[32];
  __shared__ uint32_t cand[kPfWG / 64][kMaxRouteExperts];
  __shared__ uint32_t xkey[kPfWG / 64][kMaxRouteExperts];  // 0, or an exactly summed expert's key (cleared after)
  if (threadIdx.x < 32) tab[threadIdx.x] = kExp2Tab[threadIdx.x];
  for (uint32_t i = threadIdx.x; i < (kPfWG / 64) * kMaxRouteExperts; i += kPfWG) (&xkey[0][0])[i] = 0u;
  __syncthreads();
  const uint32_t t = blockIdx.x * (kPfWG / 64) + wave_id(), lane = lane_id(), wv = wave_id();
  if (t >= T) return;
  float *lg = logits + (uint64_t)t * (E + 1);
  uint32_t key[kRoutePer], id[kRoutePer], my_id, my_key;
  route_load<false>(lg, E, lane, key, id);
  // The bound: the sum's rounding (gamma ||W||max ||x||) and the fp32 rounding of the sum and of the bias add.
  uint32_t mk = 0;
#pragma unroll
  for (int i = 0; i < kRoutePer; i++) mk = max(mk, lane + 64 * i < E ? float_key(fabsf(key_float(key[i]))) : 0u);
  const double labs = (double)key_float(wave_max_u32(mk));
  const double B = (double)gamma_rmax * (double)xn[t] + 0x1p-22 * (labs + (double)bias_max) + 1e-30;
  // The K + 1 largest (lane r < K + 1: rank r), on a copy of the keys.
  const uint32_t K1 = K < E ? K + 1 : K;
  {
    uint32_t kc[kRoutePer], ic[kRoutePer];
#pragma unroll
    for (int i = 0; i < kRoutePer; i++) kc[i] = key[i], ic[i] = id[i];
    route_select(kc, ic, K1, lane, &my_id, &my_key);
  }
  const double v = (double)key_float(my_key);
  const double nxt = __shfl_down(v, 1, 64), prv = __shfl_up(v, 1, 64);
  // Rank r's order against rank r + 1 is open when their intervals (each +- B) meet.
  const bool open = lane + 1 < K1 && !(v - nxt > 2.0 * B);
  if (__ballot(open) != 0ull) {
    // The experts whose place is open: a ranked one whose interval meets a neighbour's, and, when the K-th place is
    // open, every expert ranked after the K-th whose interval reaches the K-th's. The others keep their approximate
    // logits: each is more than 2 B from every expert on one side of it, so its order against all of them stands.
    const bool amb = lane < K1 && (open || (lane >= 1 && !(prv - v > 2.0 * B)));
    const bool kopen = __shfl((int)open, (int)K - 1, 64) != 0 && K < E;
    const double thr = __shfl(v, (int)K - 1, 64) - 2.0 * B;
    const uint32_t kK = __shfl(my_key, (int)K, 64), iK = __shfl(my_id, (int)K, 64);
    uint32_t nc = 0;
    {
      const uint64_t bal = __ballot(amb);
      if (amb) cand[wv][__builtin_amdgcn_mbcnt_hi((uint32_t)(bal >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)bal, 0u))] = my_id;
      nc = (uint32_t)__popcll(bal);
    }
#pragma unroll
    for (int i = 0; i < kRoutePer; i++) {
      const uint32_t e = lane + 64 * i;
      const bool after = key[i] < kK || (key[i] == kK && e > iK);  // ranked after the (K + 1)-th
      const bool c = kopen && e < E && after && (double)key_float(key[i]) >= thr;
      const uint64_t bal = __ballot(c);
      if (c) cand[wv][nc + __builtin_amdgcn_mbcnt_hi((uint32_t)(bal >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)bal, 0u))] = e;
      nc += (uint32_t)__popcll(bal);
    }
    __builtin_amdgcn_s_waitcnt(0xc07f);
    __builtin_amdgcn_wave_barrier();
    // Sixteen lanes a candidate: lane s of group j sums the row's sixteenth s in fp64 (its magnitudes too, and the
    // least exponent sum of its products), the group adds its sixteen partials in a fixed tree; exact when the
    // magnitudes' sum is below 2^(lsb + 53). x's bf16 row is read from memory (L2) by each candidate's group: staged
    // in LDS (32 KB a work-group) it measured ~1 us slower at config 4, and kept the kernel off CUs whose LDS the
    // shared expert's launches beside it hold.
    const uint4 *xs = (const uint4 *)(xb + (uint64_t)t * H);
    const uint32_t j = lane / 16, sl = lane % 16, H16 = H / 16;  // H16 / 8 pieces of 16 B a lane
    for (uint32_t c0 = 0; c0 < nc; c0 += 4) {
      const uint32_t ci = c0 + j, e = cand[wv][min(ci, nc - 1)];
      const uint4 *wr = (const uint4 *)(W + (uint64_t)e * H + sl * H16);
      const uint4 *xr = xs + sl * H16 / 8;
      // Four chains (piece q % 4): when the sum is exact (checked below) every order gives it, so the chains and the
      // tree that joins them need not follow k.
      double acc4[4] = {0.0, 0.0, 0.0, 0.0}, mag4[4] = {0.0, 0.0, 0.0, 0.0};
      uint32_t emin = 0xffffffffu;  // the least sum of the two exponent fields of a product, two 16-bit halves
      for (uint32_t k0 = 0; k0 < H16 / 8; k0 += 16) {  // sixteen pieces of the row in flight at a time
        uint4 a[16];
#pragma unroll
        for (int q = 0; q < 16; q++) a[q] = k0 + q < H16 / 8 ? wr[k0 + q] : make_uint4(0u, 0u, 0u, 0u);
#pragma unroll
        for (int q = 0; q < 16; q++) {
          if (k0 + q >= H16 / 8) break;
          const uint4 bq = xr[k0 + q];
          const uint32_t aw[4] = {a[q].x, a[q].y, a[q].z, a[q].w}, bw[4] = {bq.x, bq.y, bq.z, bq.w};
#pragma unroll
          for (int i = 0; i < 4; i++) {
            // Each half's exponent fields (at most 255 each) added, the halves apart (no carry between them); a
            // zero or subnormal value counts as exponent 0 (its lsb is at least that low: a safe underestimate).
            const uint32_t es = ((aw[i] >> 7) & 0x00ff00ffu) + ((bw[i] >> 7) & 0x00ff00ffu);
            emin = __builtin_bit_cast(uint32_t, __builtin_elementwise_min(__builtin_bit_cast(u16x2_t, emin),
                                                                          __builtin_bit_cast(u16x2_t, es)));
            const double p0 = (double)__uint_as_float(aw[i] << 16) * (double)__uint_as_float(bw[i] << 16);
            const double p1 = (double)__uint_as_float(aw[i] & 0xffff0000u) * (double)__uint_as_float(bw[i] & 0xffff0000u);
            acc4[q % 4] = __dadd_rn(__dadd_rn(acc4[q % 4], p0), p1);
            mag4[q % 4] = __dadd_rn(__dadd_rn(mag4[q % 4], fabs(p0)), fabs(p1));
          }
        }
      }
      double acc = __dadd_rn(__dadd_rn(acc4[0], acc4[1]), __dadd_rn(acc4[2], acc4[3]));
      double mag = __dadd_rn(__dadd_rn(mag4[0], mag4[1]), __dadd_rn(mag4[2], mag4[3]));
      uint32_t em = min(emin & 0xffffu, emin >> 16);
#pragma unroll
      for (int o = 1; o < 16; o <<= 1) {
        acc = __dadd_rn(acc, __shfl_xor(acc, o, 64));
        mag = __dadd_rn(mag, __shfl_xor(mag, o, 64));
        em = min(em, (uint32_t)__shfl_xor((int)em, o, 64));
      }
      // Every product is a multiple of 2^(em - 268) (exponent fields less 127 each, less 7 mantissa bits each), and of
      // 2^(rlsb + xlsb): exact when the magnitudes' sum stays below 2^53 times the larger of the two.
      const int lsb = max((int)em - 268, rlsb[e] + xlsb[t]);
      const bool exact_ok = mag * (1.0 + 0x1p-40) < ldexp(1.0, lsb + 53);
      float lgv = (float)acc;
      if (!exact_ok && sl == 0 && ci < nc) lgv = exact_logit_chain(W, xb, H, e, t);
      if (sl == 0 && ci < nc) xkey[wv][e] = float_key(bias ? __fadd_rn(lgv, bias[e]) : lgv);
    }
    __builtin_amdgcn_s_waitcnt(0xc07f);
    __builtin_amdgcn_wave_barrier();
#pragma unroll
    for (int i = 0; i < kRoutePer; i++) {
      const uint32_t e = lane + 64 * i;
      if (e < E && xkey[wv][e] != 0u) key[i] = xkey[wv][e], xkey[wv][e] = 0u;
    }
    if (lane == 0) atomicAdd(cnt_exact, 1u);
    uint32_t kc[kRoutePer], ic[kRoutePer];
#pragma unroll
    for (int i = 0; i < kRoutePer; i++) kc[i] = key[i], ic[i] = id[i];
    route_select(kc, ic, K, lane, &my_id, &my_key);
  }
  float mx, inv;
  route_norm(key, E, lane, tab, &mx, &inv);
  const float wk = route_weight(my_key, mx, inv, K, lane, tab);
  if (lane < K) {
    ids[(uint64_t)t * K + lane] = (int32_t)my_id;
    w[(uint64_t)t * K + lane] = wk;
    atomicOr(&masks[(uint64_t)(t / 64) * E + my_id], 1ull << (t % 64));
  }
}

// ---------------------------------------------------------------------------------------------------------------
// Dispatch (p_moe_count / p_moe_scan / p_moe_fill, prompt.cl:682-738): a counting sort of the T k assignments by
// expert, stable (token order within an expert; the reference's fill takes atomic order). An expert takes at most one
// assignment a token, so a 64-bit mask per (64-token window, expert) of the tokens that chose it gives both the counts
// and each assignment's rank inside its window. Two steps:
//   the masks  built by pf_topk as it selects (global atomics on masks the router's gate-row work-groups cleared),
//              or, for pre-routed ids, by pf_masks (one work-group a window, LDS atomics, written out whole);
//   pf_place   one work-group a window: the counts, the experts' bases and the window's starts from the masks, then
//              position = start of (window, expert) + the lower bits of the mask; perm and inv; the MoeTile records.

constexpr uint32_t kDispWG = 512;

__global__ void __launch_bounds__(kDispWG) pf_masks(const int32_t *ids, uint32_t T, uint32_t K, uint32_t E,
                                                    unsigned long long *masks) {
  __shared__ unsigned long long m[512];
  const uint32_t w = blockIdx.x, t0 = 64 * w, tid = threadIdx.x;
  m[tid] = 0ull;
  __syncthreads();
  const uint32_t a0 = t0 * K, a1 = min(T, t0 + 64) * K;
  for (uint32_t a = a0 + tid; a < a1; a += kDispWG) {
    const int32_t id = ids[a];  // < 0: no assignment (a pre-routed call's token with fewer jobs)
    if (id >= 0) atomicOr(&m[(uint32_t)id], 1ull << (a / K - t0));
  }
  __syncthreads();
  if (tid < E) masks[(uint64_t)w * E + tid] = m[tid];
}

// An inclusive scan of v over the work-group's 512 threads (wave scans, then the waves' totals).
__device__ __forceinline__ uint32_t block_scan512(uint32_t v, uint32_t *wsum) {
  const uint32_t lane = threadIdx.x & 63u, wv = threadIdx.x >> 6;
#pragma unroll
  for (uint32_t o = 1; o < 64; o <<= 1) {
    const uint32_t x = __shfl_up(v, o, 64);
    if (lane >= o) v += x;
  }
  if (lane == 63) wsum[wv] = v;
  __syncthreads();
  uint32_t add = 0;
  for (uint32_t i = 0; i < wv; i++) add += wsum[i];
  __syncthreads();
  return v + add;
}

constexpr uint32_t kScanBatch = 32;  // window masks a thread holds at once (all of them up to 2048 tokens)

// One work-group a window. Thread e counts expert e's assignments in every window (the masks' popcounts, all loaded
// before the first is used) and in the windows before this one; a scan over experts gives each expert's base, so the
// (window, expert) start is base + the earlier windows' count. The window's assignments are then placed at that start
// plus the popcount of the lower mask bits; window 0's work-group also writes the MoeTile records (at most MOE_TILE
// rows) and their count.
__global__ void __launch_bounds__(kDispWG) pf_place(const int32_t *ids, uint32_t T, uint32_t K, uint32_t E,
                                                    uint32_t nwin, const unsigned long long *masks, MoeTile *tiles,
                                                    uint32_t *ntiles, uint32_t *perm, uint32_t *inv) {
  __shared__ uint32_t wsum[kDispWG / 64], start[kDispWG];
  __shared__ unsigned long long mine[kDispWG];
  const uint32_t w = blockIdx.x, e = threadIdx.x, ec = min(e, E - 1);
  uint32_t c = 0, before = 0;
  for (uint32_t j0 = 0; j0 < nwin; j0 += kScanBatch) {
    // Unconditional loads (clamped indices, masked after), so that all are in flight before the first is used.
    unsigned long long mm[kScanBatch];
#pragma unroll
    for (uint32_t j = 0; j < kScanBatch; j++) mm[j] = masks[(uint64_t)min(j0 + j, nwin - 1) * E + ec];
#pragma unroll
    for (uint32_t j = 0; j < kScanBatch; j++) {
      const uint32_t n = e < E && j0 + j < nwin ? (uint32_t)__popcll(mm[j]) : 0u;
      c += n;
      before += j0 + j < w ? n : 0u;
    }
  }
  const uint32_t base = block_scan512(c, wsum) - c;
  start[e] = base + before;
  mine[e] = e < E ? masks[(uint64_t)w * E + e] : 0ull;
  if (w == 0) {
    const uint32_t nt = (c + MOE_TILE - 1) / MOE_TILE, t0 = block_scan512(nt, wsum) - nt;
    if (e < E)
      for (uint32_t i = 0; i < nt; i++) {
        MoeTile m;
        m.expert = e, m.slot = e, m.start = base + MOE_TILE * i, m.count = min((uint32_t)MOE_TILE, c - MOE_TILE * i);
        tiles[t0 + i] = m;
      }
    if (e == E - 1) *ntiles = t0 + nt;
  }
  __syncthreads();
  const uint32_t t0 = 64 * w, a0 = t0 * K, a1 = min(T, t0 + 64) * K;
  for (uint32_t a = a0 + e; a < a1; a += kDispWG) {
    const int32_t id = ids[a];
    if (id < 0) continue;
    const uint32_t t = a / K - t0;
    const uint32_t pos = start[id] + (uint32_t)__popcll(mine[id] & ((1ull << t) - 1ull));
    perm[pos] = a;
    inv[a] = pos;
  }
}

// ---------------------------------------------------------------------------------------------------------------
// Expert GEMMs on int8 MFMA.
//
struct PfGemm {
  const MoeTile *tiles;    // routed: the dispatch's tiles
  const uint32_t *ntiles;
  uint32_t shared_T;       // > 0: the shared expert over tokens 0 .. shared_T - 1 in order (implicit tiles)
  const uint32_t *perm;    // routed gate/up: position -> assignment (token = assignment / K)
  uint32_t K;
  const uint8_t *act;      // activation units: by token (gate/up) or by position (down)
  uint32_t act_by_pos;
  const uint8_t *mat;      // expert e's matrix at mat + e * stride; up at + up_off
  uint64_t stride, up_off;
  float *out;              // position p's outputs at out + p * out_ld
  uint32_t out_ld;
  float limit;
  uint32_t row_blocks;     // row blocks a tile (the 1-D grid is tiles x row_blocks)
  uint32_t rb_span;        // pf_gemm16 Q4_K down: consecutive 64-row blocks a work-group (> 1 only when U <= 2)
  uint32_t U;              // 256-value units of K (a partial last one padded with zeros)
  const uint8_t *codebooks;  // the caller's codebooks (QGRID layout) for IQ3_XXS and IQ2_S
};

// Rows of one grid.y step of the (tiles x row groups) grid the host computes: 64 of gate and of up, or 128 of down.
// pf_gemm16 splits each into row blocks of 32 gate + 32 up rows, or 64 down rows, one work-group each.
template <bool kGU>
constexpr uint32_t gemm_rows() { return kGU ? 64 : 128; }

// A work-group's kPos positions' activation units go into LDS by direct global-to-LDS loads: LDS holds 21 pieces of
// 16 B a position (kActLds = 336), so load i fills pieces 64 i .. 64 i + 63 contiguously, lane l piece 64 i + l, of
// position (64 i + l) / 21. Pieces 0-19 are the 320-byte global unit verbatim (with the split block sums at kActSplitH
// for q8_K). The loads are dealt to the waves (load i to wave i % kWaves); a wave's global offsets are the same for
// every unit but for + u kActBytes, so they are worked out once (plan). Piece 20 (padding) and positions without a
// row load the first unit instead: the bytes land where no operand is read (padding, or MFMA columns never stored),
// and every lane issues its loads, without branches.
template <uint32_t kPos, uint32_t kWaves>
struct Dma {
  static constexpr uint32_t kLoads = kPos * kActLds / 16 / 64, kPer = (kLoads + kWaves - 1) / kWaves;
  static_assert(kActLds == 21 * 16 && kPos * 21 % 64 == 0, "activation pieces");
  uint32_t off[kPer];
  // The calling wave's global offsets (unit 0) of its loads, from the positions' rows arow[] (0xffffffff: none).
  __device__ __forceinline__ void plan(const uint32_t *arow, uint32_t U) {
#pragma unroll
    for (uint32_t k = 0; k < kPer; k++) {
      const uint32_t i = wave_id() + kWaves * k, piece = 64 * i + lane_id(), pos = piece / 21, c = piece % 21;
      const uint32_t ar = i < kLoads ? arow[pos] : 0xffffffffu;
      off[k] = c < 20 && ar != 0xffffffffu ? ar * U * kActBytes + 16 * c : 0u;
    }
  }
  // As load, but every wave issues kPer loads, those past kLoads into dump (1 KB of LDS no one reads): no branches,
  // and the same count of loads in every wave, so that a wait can leave exactly the later units' loads in flight.
  // Buffer loads on a resource over act (uniform base, the lane's 32-bit offset, the unit's scalar offset) and LDS
  // destinations from the wave's uniform index: no vector address arithmetic a load.
  __device__ __forceinline__ void load_all(__amdgpu_buffer_rsrc_t act, uint32_t u, uint8_t *buf, uint8_t *dump) const {
    const uint32_t w = (uint32_t)__builtin_amdgcn_readfirstlane(wave_id());
#pragma unroll
    for (uint32_t k = 0; k < kPer; k++) {
      const uint32_t i = w + kWaves * k;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(act, (__attribute__((address_space(3))) void *)(i < kLoads ? buf + 64 * 16 * i : dump),
                                               16, off[k], u * kActBytes, 0, 0);
    }
  }
  // Unit u of the planned positions into LDS at buf (the calling wave's share of the loads). The caller waits
  // (s_waitcnt vmcnt(0)) and synchronises before reading.
  __device__ __forceinline__ void load(const uint8_t *act, uint32_t u, uint8_t *buf) const {
    const uint8_t *base = act + (uint64_t)u * kActBytes;
#pragma unroll
    for (uint32_t k = 0; k < kPer; k++) {
      const uint32_t i = wave_id() + kWaves * k;
      if (i < kLoads)
        __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void *)(base + off[k]),
                                         (__attribute__((address_space(3))) void *)(buf + 64 * 16 * i), 16, 0, 0);
    }
  }
};


// The s_waitcnt immediate (gfx9 encoding) that waits until at most n vector memory loads are outstanding and
// leaves the other counters alone.
constexpr uint32_t vm_wait(uint32_t n) { return (n & 15u) | ((n >> 4) << 14) | (7u << 4) | (15u << 8); }

// The decoded operands as the outputs of an empty volatile asm with a memory clobber: the decode is done there (it
// cannot sink below to its uses), and the next unit's loads, issued after it, cannot rise above it. Otherwise the
// compiler moves the decode past the loads, the old and new raw words are live together, and the waits it inserts
// for them cover the loads just issued.
__device__ __forceinline__ void pin(Q4kA &a) {
  asm volatile("" : "+v"(a.lo[0]), "+v"(a.lo[1]), "+v"(a.lo[2]), "+v"(a.lo[3]), "+v"(a.hi[0]), "+v"(a.hi[1]),
               "+v"(a.hi[2]), "+v"(a.hi[3]), "+v"(a.mn), "+v"(a.d[0]), "+v"(a.d[1]), "+v"(a.d[2]), "+v"(a.d[3]),
               "+v"(a.dmin[0]), "+v"(a.dmin[1]), "+v"(a.dmin[2]), "+v"(a.dmin[3]) :: "memory");
}
__device__ __forceinline__ void pin(Q4kRaw &r) {
  asm volatile("" : "+v"(r.qs[0]), "+v"(r.qs[1]), "+v"(r.qs[2]), "+v"(r.qs[3]), "+v"(r.sc[0]), "+v"(r.sc[1]),
               "+v"(r.sc[2]), "+v"(r.dm[0]), "+v"(r.dm[1]), "+v"(r.dm[2]), "+v"(r.dm[3]) :: "memory");
}

// A raw buffer resource over p (wave-uniform), the whole 32-bit offset range.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t uniform_rsrc(const void *p) {
  const uint64_t b = (uint64_t)p;
  const uint32_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)(b >> 32));
  const uint32_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)b);
  return __builtin_amdgcn_make_buffer_rsrc((void *)(((uint64_t)hi << 32) | lo), 0, 0xffffffffu, 0x00020000u);
}

// Q4kRaw's loads for gate and up as buffer loads on the wave's 16-row tiles: a resource over each tile, the lane's
// three 32-bit offsets (the same for both) worked out once, each field's and unit's offset scalar (the same bytes as
// Q4kRaw::load_qs / load_meta).
struct Q4kBuf {
  const uint8_t *base[2];  // the resources are made at each load (scalar work the compiler keeps out of the loop)
  uint32_t nl, lq, ls, ld;
  __device__ __forceinline__ void init(const uint8_t *gate, const uint8_t *up, uint32_t U, uint32_t row0, uint32_t lane) {
    const uint32_t g = lane / 16, rr = row0 % kTileRows;
    const uint64_t t = (uint64_t)(row0 / kTileRows) * tile_bytes(QT_Q4_K, U);
    nl = kTileRows * U;
    base[0] = gate + t, base[1] = up + t;
    lq = (g / 2) * nl * 16 + (rr + lane % 16) * 16 + 8 * (g % 2);
    ls = (rr + lane % 16) * 4;
    ld = (rr + 4 * g) * 4;
  }
  // The same rows of the next 64-row tile.
  __device__ __forceinline__ void next_block(uint32_t U) {
    base[0] += tile_bytes(QT_Q4_K, U), base[1] += tile_bytes(QT_Q4_K, U);
  }
  __device__ __forceinline__ void load_qs(uint32_t m, Q4kRaw &w, uint32_t u) const {
#pragma unroll
    for (uint32_t c = 0; c < 4; c++) {
      const auto v = __builtin_amdgcn_raw_buffer_load_b64(uniform_rsrc(base[m]), lq, (q4_kt::kQs / 16 + 2 * c) * nl * 16 + u * kTileRows * 16, 0);
      w.qs[c] = make_uint2(v[0], v[1]);
    }
  }
  __device__ __forceinline__ void load_meta(uint32_t m, Q4kRaw &w, uint32_t u) const {
#pragma unroll
    for (uint32_t i = 0; i < 3; i++)
      w.sc[i] = __builtin_amdgcn_raw_buffer_load_b32(uniform_rsrc(base[m]), ls, (q4_kt::kScales + 4 * i) * nl + u * kTileRows * 4, 0);
    const auto v = __builtin_amdgcn_raw_buffer_load_b128(uniform_rsrc(base[m]), ld, q4_kt::kDm * nl + u * kTileRows * 4, 0);
    w.dm[0] = v[0], w.dm[1] = v[1], w.dm[2] = v[2], w.dm[3] = v[3];
  }
};

// Iq3sRaw's loads for gate and up as buffer loads on the wave's 16-row tiles, as Q4kBuf's: the lane's offsets worked
// out once, each field's, piece's and unit's offset scalar (the same bytes as Iq3sRaw::load; the four D rows' d words
// are consecutive, one 8-byte load).
struct Iq3sBuf {
  const uint8_t *base[2];
  uint32_t nl, lq, la, ld;
  __device__ __forceinline__ void init(const uint8_t *gate, const uint8_t *up, uint32_t U, uint32_t row0, uint32_t lane) {
    const uint32_t g = lane / 16, rr = row0 % kTileRows;
    const uint64_t t = (uint64_t)(row0 / kTileRows) * tile_bytes(QT_IQ3_S, U);
    nl = kTileRows * U;
    base[0] = gate + t, base[1] = up + t;
    la = rr + lane % 16;      // the A row's pair index within a unit
    lq = la * 16 + 4 * (g / 2);
    ld = rr + 4 * g;          // the first D row's
  }
  __device__ __forceinline__ void load(uint32_t m, Iq3sRaw &w, uint32_t u) const {
    const uint32_t pu = u * kTileRows;
#pragma unroll
    for (uint32_t ib = 0; ib < 8; ib++)
      w.qs[ib] = __builtin_amdgcn_raw_buffer_load_b32(uniform_rsrc(base[m]), lq + 8 * (ib % 2), ((ib / 2) * nl + pu) * 16, 0);
#pragma unroll
    for (uint32_t p = 0; p < 2; p++) {
      const auto v = __builtin_amdgcn_raw_buffer_load_b128(uniform_rsrc(base[m]), la * 16, iq3_st::kSigns * nl + (p * nl + pu) * 16, 0);
      w.sg[4 * p] = v[0], w.sg[4 * p + 1] = v[1], w.sg[4 * p + 2] = v[2], w.sg[4 * p + 3] = v[3];
    }
#pragma unroll
    for (uint32_t p = 0; p < 2; p++)
      w.qh[p] = __builtin_amdgcn_raw_buffer_load_b32(uniform_rsrc(base[m]), la * 4, iq3_st::kQh * nl + (p * nl + pu) * 4, 0);
#pragma unroll
    for (uint32_t i = 0; i < 4; i++)
      w.sc[i] = __builtin_amdgcn_raw_buffer_load_b32(uniform_rsrc(base[m]), (ld + i) * 4, iq3_st::kScales * nl + pu * 4, 0);
    const auto d = __builtin_amdgcn_raw_buffer_load_b64(uniform_rsrc(base[m]), ld * 2, iq3_st::kD * nl + pu * 2, 0);
    w.dh[0] = d[0] & 0xffffu, w.dh[1] = d[0] >> 16, w.dh[2] = d[1] & 0xffffu, w.dh[3] = d[1] >> 16;
  }
};

// A work-group barrier without __syncthreads' fence (which would wait for every load in flight): LDS reads done, then
// s_barrier, with compiler barriers either side so that no LDS access moves across it.
__device__ __forceinline__ void unit_barrier() {
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// Q4_K, IQ3_S and Q8_0 on 16 x 16 int8 MFMA tiles (mfma_q4k.h, the decode path's tile; mfma_iq3s.h; mfma_q8_0.h):
// wave w takes 16 weight rows (gate/up: matrix w / 2, rows 16 (w % 2) .. of the work-group's 32 of each; down: rows
// 16 w .. of its 64) against the tile's positions in 16-position tiles (only those holding positions run), unit by
// unit: the same integers and fp32 steps as UnitQ4_K::term / UnitIQ3_S::term / UnitQ8_0::term, units added in
// sequence; three work-groups share a CU.
template <uint32_t kType, bool kGU>
__global__ void __launch_bounds__(kPfWG) __attribute__((amdgpu_waves_per_eu(3))) pf_gemm16(PfGemm g) {
  const uint32_t U = g.U;
  constexpr uint32_t kRows = kGU ? 32 : 64;
  // Two activation buffers filled by direct global-to-LDS loads (no registers held), the next unit's issued before
  // the current unit's MFMAs and waited for after them: one barrier a unit, three waves a SIMD.
  __shared__ __align__(16) uint8_t abuf[2][64 * kActLds];
  __shared__ __align__(16) uint8_t dump[64 * 16];
  // Up sums [row][position], written after the unit loop's last barrier: they reuse the activation buffer.
  static_assert(32 * 65 * sizeof(float) <= 64 * kActLds, "ub must fit in one activation buffer");
  float(*ub)[65] = reinterpret_cast<float(*)[65]>(&abuf[0][0]);
  __shared__ uint32_t arow_lds[64];
  __shared__ uint64_t tab[32];
  __shared__ uint32_t grid_lds[kType == QT_IQ3_S ? 512 : kType == QT_IQ3_XXS ? 256 : kType == QT_IQ2_S ? 2048 : 1];
  using Raw = std::conditional_t<
      kType == QT_IQ3_S, Iq3sRaw,
      std::conditional_t<
          kType == QT_IQ3_XXS, Iq3xxsRaw,
          std::conditional_t<
              kType == QT_IQ2_S, Iq2sRaw,
              std::conditional_t<
                  kType == QT_Q8_0, Q80Raw,
                  std::conditional_t<
                      kType == QT_IQ4_NL, Iq4nlRaw,
                      std::conditional_t<
                          kType == QT_Q2_0, Q20Raw,
                          std::conditional_t<
                              kType == QT_IQ4_XS, Iq4xsRaw,
                              std::conditional_t<kType == QT_Q5_K, Q5kRaw,
                                                 std::conditional_t<kType == QT_Q6_K, Q6kRaw, Q4kRaw>>>>>>>>>;
  // 1-D grid of (tile, row block) pairs, the row block fastest in the XCD-aware logical index over the pairs that
  // exist (the grid is sized for the most tiles a dispatch can make).
  const uint32_t nrb = g.row_blocks;
  const uint32_t ntl = g.shared_T ? (g.shared_T + MOE_TILE - 1) / MOE_TILE : *g.ntiles, n = ntl * nrb;
  if (blockIdx.x >= n) return;
  const uint32_t L = xcd_logical(blockIdx.x, n);
  if (L >= n) return;
  const uint32_t tile_i = L / nrb, rb = L % nrb;
  // Down: R consecutive row blocks, one after another on the same positions. With U <= 2 (the host's condition for
  // R > 1) every unit's activations stay in their LDS buffer after the first row block, so only its weights load.
  // Q4_K only: the other types' forms spill with the row-block loop.
  constexpr bool kWalk = !kGU && kType == QT_Q4_K;
  const uint32_t R = kWalk && U <= 2 ? g.rb_span : 1u;  // (the host sets rb_span 1 for U > 2 too)
  uint32_t start, count, e;
  if (g.shared_T) {
    start = MOE_TILE * tile_i;
    if (start >= g.shared_T) return;
    count = min((uint32_t)MOE_TILE, g.shared_T - start), e = 0;
  } else {
    if (tile_i >= *g.ntiles) return;
    const MoeTile tl = g.tiles[tile_i];
    start = tl.start, count = tl.count, e = tl.slot;
  }
  const uint32_t tid = tid_fresh(), w = wave_id();
  if (tid < 32) tab[tid] = kExp2Tab[tid];
  if constexpr (kType == QT_IQ3_S)
    for (uint32_t i = tid; i < 512; i += kPfWG) grid_lds[i] = kIq3sGridPf[i];
  if constexpr (kType == QT_IQ3_XXS || kType == QT_IQ2_S) {
    const uint32_t *src = (const uint32_t *)(g.codebooks + (kType == QT_IQ2_S ? QGRID_IQ2S : QGRID_IQ3XXS));
    for (uint32_t i = tid; i < (kType == QT_IQ2_S ? 2048u : 256u); i += kPfWG) grid_lds[i] = src[i];
  }
  if (tid < 64) {
    const uint32_t pos = start + tid;
    arow_lds[tid] = tid < count ? (g.act_by_pos ? pos : (g.perm ? g.perm[pos] / g.K : pos)) : 0xffffffffu;
  }
  __syncthreads();
  const uint32_t mat = kGU ? (w >> 1) : 0u;
  const uint32_t row0 = rb * R * kRows + (kGU ? 16 * (w & 1) : 16 * w);
  const uint8_t *M = g.mat + (uint64_t)e * g.stride + (mat ? g.up_off : 0);
  const uint32_t npt = (count + 15) / 16;  // 16-position tiles with positions
  Dma<64, 4> dma;
  dma.plan(arow_lds, U);
  const __amdgpu_buffer_rsrc_t act_r = uniform_rsrc(g.act);
  Q4kBuf wb;  // Q4_K's weight loads as buffer loads (the other types through their Raw::load)
  if constexpr (kType == QT_Q4_K) wb.init(M, M, U, row0, lane_id());
  // Unit u of the wave's rows from row rows0 (Q4_K: from wb's tile, which next_block moves on a row block).
  const auto load_w = [&](Raw &r, uint32_t u, uint32_t rows0) {
    if constexpr (kType == QT_Q4_K)
      wb.load_qs(0, r, u), wb.load_meta(0, r, u);
    else
      r.load(M, U, rows0, u, lane_id());
  };
  Raw raw;
  load_w(raw, 0, row0);
  dma.load_all(act_r, 0, &abuf[0][0], dump);
  __builtin_amdgcn_s_waitcnt(vm_wait(0));
  unit_barrier();
  float acc[4][4];
#pragma unroll
  for (int pt = 0; pt < 4; pt++)
#pragma unroll
    for (int i = 0; i < 4; i++) acc[pt][i] = 0.0f;
  // buf (read) and nbuf (filled) as restrict pointers: the compiler then knows the reads of buf need not wait for the
  // global-to-LDS loads into nbuf (without it, each position tile's first LDS read waited for every load in flight).
  // Step (r, u): unit u of row block r. The next step's weights are unit u + 1's, or the next row block's unit 0.
  const auto body = [&](uint32_t r, uint32_t u, const uint8_t *__restrict__ buf, uint8_t *__restrict__ nbuf) {
    // Q4_K decodes the unit's raw words first and loads the next unit's into the same registers; the other types read
    // theirs in the MFMAs and load the next unit's into a second set.
    constexpr bool kInPlace = kType == QT_Q4_K || kType == QT_Q5_K;  // Q5_K: registers for one unit's words only
    const bool more = kWalk ? u + 1 < U || r + 1 < R : u + 1 < U;
    const uint32_t nu = !kWalk || u + 1 < U ? u + 1 : 0u, nrow = row0 + (!kWalk || u + 1 < U ? r : r + 1) * kRows;
    if constexpr (kType == QT_Q4_K)
      if (u + 1 == U && r + 1 < R) wb.next_block(U);  // the raw words of (r, u) are loaded: move to block r + 1
    Raw next;
    if (r == 0 && u + 1 < U) dma.load_all(act_r, u + 1, nbuf, dump);
    if constexpr (!kInPlace)
      if (more) load_w(next, nu, nrow);
    if constexpr (block_scaled(kType)) {
      // Block by block: one MFMA a position tile (IQ2_S, Q6_K: one a half block, the other half's A lanes zero), its
      // D times the row's block scale added to the unit's integer sum in block order; then kFactor ((d ad) isum) as
      // UnitIQ3_S / UnitIQ3_XXS / UnitIQ2_S / UnitIQ4_XS / UnitQ6_K::term, or Q5_K's fma(d ad, isum, -((dmin ad)
      // imin)) with imin from the positions' block sums (UnitQ4_K::term).
      raw.prep(lane_id());
      int isum[4][4];
#pragma unroll
      for (int pt = 0; pt < 4; pt++)
#pragma unroll
        for (int i = 0; i < 4; i++) isum[pt][i] = 0;
#pragma unroll
      for (uint32_t ib = 0; ib < 8; ib++) {
        const uint32_t bofs = mfma_code_off(4 * ib + lane_id() / 16);  // the lane's 8 codes of block ib
        const long aw = raw.a_block(ib, lane_id(), grid_lds);
        if constexpr (Raw::kHalves == 2) {
          const bool lo = lane_id() < 32;
          const long a0 = lo ? aw : 0, a1 = lo ? 0 : aw;
          int l0[4], l1[4];
#pragma unroll
          for (uint32_t i = 0; i < 4; i++) l0[i] = raw.ls(i, ib, 0), l1[i] = raw.ls(i, ib, 1);
#pragma unroll
          for (uint32_t pt = 0; pt < 4; pt++) {
            if (pt < npt) {
              const long bw = *(const long *)(buf + (16 * pt + lane_id() % 16) * kActLds + bofs);
              const v4i_t d0 = __builtin_amdgcn_mfma_i32_16x16x32_i8(a0, bw, v4i_t{0, 0, 0, 0}, 0, 0, 0);
              const v4i_t d1 = __builtin_amdgcn_mfma_i32_16x16x32_i8(a1, bw, v4i_t{0, 0, 0, 0}, 0, 0, 0);
#pragma unroll
              for (int i = 0; i < 4; i++) isum[pt][i] += l0[i] * d0[i] + l1[i] * d1[i];
            }
          }
        } else {
          int ls[4];
#pragma unroll
          for (uint32_t i = 0; i < 4; i++) ls[i] = raw.ls(i, ib);
#pragma unroll
          for (uint32_t pt = 0; pt < 4; pt++) {
            if (pt < npt) {
              const long bw = *(const long *)(buf + (16 * pt + lane_id() % 16) * kActLds + bofs);
              const v4i_t dv = __builtin_amdgcn_mfma_i32_16x16x32_i8(aw, bw, v4i_t{0, 0, 0, 0}, 0, 0, 0);
#pragma unroll
              for (int i = 0; i < 4; i++) isum[pt][i] += ls[i] * dv[i];
            }
          }
        }
        __builtin_amdgcn_sched_barrier(0);  // one block's operands live at a time
      }
#pragma unroll
      for (uint32_t pt = 0; pt < 4; pt++) {
        if (pt < npt) {
          const uint8_t *unit = buf + (16 * pt + lane_id() % 16) * kActLds;
          const float ad = *(const float *)(unit + kActScales);
          if constexpr (Raw::kMin) {
            int bs[8];
#pragma unroll
            for (uint32_t j = 0; j < 8; j++)  // lo_j + 64 hi_j from the f16 split (exact integers)
              bs[j] = (int)h2f(*(const uint16_t *)(unit + kActSplitH + 2 * j)) +
                      (int)h2f(*(const uint16_t *)(unit + kActSplitH + 16 + 2 * j));
#pragma unroll
            for (int i = 0; i < 4; i++) {
              int imin = 0;
#pragma unroll
              for (uint32_t j = 0; j < 8; j++) imin += raw.mn(i, j) * bs[j];
              const float dd = __fmul_rn(h2f((uint16_t)raw.dh[i]), ad), dm = __fmul_rn(raw.dmin(i), ad);
              const float t = __builtin_fmaf(dd, (float)isum[pt][i], -__fmul_rn(dm, (float)imin));
              acc[pt][i] = __fadd_rn(acc[pt][i], t);
            }
          } else {
#pragma unroll
            for (int i = 0; i < 4; i++) {
              float t = __fmul_rn(__fmul_rn(h2f((uint16_t)raw.dh[i]), ad), (float)isum[pt][i]);
              if constexpr (Raw::kFactor != 1.0f) t = __fmul_rn(Raw::kFactor, t);
              acc[pt][i] = __fadd_rn(acc[pt][i], t);
            }
          }
        }
      }
      if constexpr (kInPlace)
        if (more) load_w(raw, nu, nrow);
    } else if constexpr (q8_family(kType)) {
      // Block by block: one MFMA a position tile, the block's term (d_w d_a) dot; the eight terms of the unit as the
      // pairwise tree ((c0 + c1) + (c2 + c3)) + ((c4 + c5) + (c6 + c7)), then added to the row's sum.
      raw.widen(lane_id());  // IQ4_NL, Q2_0: codes from the raw bytes
      float q[3][4][4];  // the tree's pending partial sums: q[level][pt][row]
#pragma unroll
      for (uint32_t j = 0; j < 8; j++) {
        const uint32_t bofs = mfma_code_off(4 * j + lane_id() / 16);  // the lane's 8 codes of block j
        float dw[4];
#pragma unroll
        for (uint32_t i = 0; i < 4; i++) dw[i] = raw.d(i, j);
#pragma unroll
        for (uint32_t pt = 0; pt < 4; pt++) {
          if (pt < npt) {
            const uint8_t *unit = buf + (16 * pt + lane_id() % 16) * kActLds;
            const v4i_t dv = __builtin_amdgcn_mfma_i32_16x16x32_i8(raw.qs[j], *(const long *)(unit + bofs),
                                                                  v4i_t{0, 0, 0, 0}, 0, 0, 0);
            const float as = *(const float *)(unit + kActScales + 4 * j);
#pragma unroll
            for (int i = 0; i < 4; i++) {
              float c = __fmul_rn(__fmul_rn(dw[i], as), (float)dv[i]);
              if ((j & 1) == 0) {
                q[0][pt][i] = c;
              } else {
                c = __fadd_rn(q[0][pt][i], c);
                if ((j & 2) == 0) {
                  q[1][pt][i] = c;
                } else {
                  c = __fadd_rn(q[1][pt][i], c);
                  if ((j & 4) == 0)
                    q[2][pt][i] = c;
                  else
                    acc[pt][i] = __fadd_rn(acc[pt][i], __fadd_rn(q[2][pt][i], c));
                }
              }
            }
          }
        }
        __builtin_amdgcn_sched_barrier(0);  // one block's operands live at a time
      }
    } else {
      Q4kA a;
      pin(raw);  // the decode starts after the previous unit's barrier ...
      a.decode<true>(raw, lane_id());
      pin(a);  // ... and ends before the next unit's loads into the raw registers
      if (more) load_w(raw, nu, nrow);
#pragma unroll
      for (uint32_t pt = 0; pt < 4; pt++) {
        if (pt < npt) {
          ActBP b;
          b.load(buf + (16 * pt + lane_id() % 16) * kActLds, lane_id());
          float t[4];
          q4k_terms_p(a, b, t);
#pragma unroll
          for (int i = 0; i < 4; i++) acc[pt][i] = __fadd_rn(acc[pt][i], t[i]);
        }
      }
    }
    if constexpr (!kInPlace)
      if (more) raw = next;
    __builtin_amdgcn_s_waitcnt(vm_wait(0));  // this wave's loads of unit u + 1 have landed ...
    // ... and every wave's, where this step loaded activations (so also every wave is done reading the buffer the
    // next step's loads refill), or, gate/up, before the up sums reuse the buffer. The other steps leave LDS as it
    // is, so the waves need not meet (down, config 4: 100 -> 95.5 us).
    if (kGU || (r == 0 && u + 1 < U)) unit_barrier();
  };
  if constexpr (!kGU) {
#pragma unroll 1
    for (uint32_t r = 0; r < R; r++) {
#pragma unroll 1
      for (uint32_t u = 0; u < U; u++) body(r, u, abuf[u & 1], abuf[(u + 1) & 1]);
      // Lane l holds rows row0 + r kRows + 4 (l / 16) + i of positions 16 pt + l % 16.
      const uint32_t l = lane_id(), r4 = 4 * (l / 16), c16 = l % 16;
#pragma unroll
      for (uint32_t pt = 0; pt < 4; pt++)
#pragma unroll
        for (int i = 0; i < 4; i++) {
          const uint32_t m = 16 * pt + c16;
          if (m < count) g.out[(uint64_t)(start + m) * g.out_ld + row0 + r * kRows + r4 + i] = acc[pt][i];
          acc[pt][i] = 0.0f;
        }
    }
  } else {
#pragma unroll 1
    for (uint32_t u = 0; u < U; u++) body(0, u, abuf[u & 1], abuf[(u + 1) & 1]);
    // Lane l holds rows row0 + 4 (l / 16) + i of positions 16 pt + l % 16.
    const uint32_t l = lane_id(), r4 = 4 * (l / 16), c16 = l % 16;

    if (mat == 1) {
#pragma unroll
      for (uint32_t pt = 0; pt < 4; pt++)
#pragma unroll
        for (int i = 0; i < 4; i++) ub[16 * (w & 1) + r4 + i][16 * pt + c16] = acc[pt][i];
    }
    __syncthreads();
    if (mat == 0) {
#pragma unroll
      for (uint32_t pt = 0; pt < 4; pt++)
#pragma unroll
        for (int i = 0; i < 4; i++) {
          const uint32_t m = 16 * pt + c16;
          if (m < count)
            g.out[(uint64_t)(start + m) * g.out_ld + row0 + r4 + i] =
                swiglu_one(acc[pt][i], ub[16 * (w & 1) + r4 + i][m], g.limit, tab);
        }
    }
  }
}

__device__ __forceinline__ void pin(Iq3sRaw &r) {
  asm volatile("" : "+v"(r.qs[0]), "+v"(r.qs[1]), "+v"(r.qs[2]), "+v"(r.qs[3]), "+v"(r.qs[4]), "+v"(r.qs[5]),
               "+v"(r.qs[6]), "+v"(r.qs[7]), "+v"(r.sg[0]), "+v"(r.sg[1]), "+v"(r.sg[2]), "+v"(r.sg[3]), "+v"(r.sg[4]),
               "+v"(r.sg[5]), "+v"(r.sg[6]), "+v"(r.sg[7]) :: "memory");
  asm volatile("" : "+v"(r.qh[0]), "+v"(r.qh[1]), "+v"(r.sc[0]), "+v"(r.sc[1]), "+v"(r.sc[2]), "+v"(r.sc[3]),
               "+v"(r.dh[0]), "+v"(r.dh[1]), "+v"(r.dh[2]), "+v"(r.dh[3]) :: "memory");
}

// Q4_K gate/up at three waves a SIMD: a unit's gate products come before its up products, so that one matrix's
// decoded operands are live at a time (150 registers; the activation operands are read from LDS once for each), and
// the activations are loaded one unit ahead into two LDS buffers (44 KB a work-group, three a CU). Wave w takes rows
// 16 w .. 16 w + 15 of gate and of up (a work-group 64 rows of each, kPos = 64 positions, four waves), so SwiGLU pairs
// gate and up in the same lane. A matrix's weights are decoded, then the registers of its raw bytes take the next
// unit's loads (buffer loads on scalar bases), which the end of the unit waits for with the activations; the
// barriers are plain ones (a fence would wait for every load in flight). The integers and fp32 steps are pf_gemm16's
// (UnitQ4_K::term), units added in sequence.
template <uint32_t kPos>
__global__ void __launch_bounds__(4 * kPos) __attribute__((amdgpu_waves_per_eu(3))) pf_gate_up_q4k(PfGemm g) {
  const uint32_t U = g.U;
  constexpr uint32_t kWaves = kPos / 16, kRows = 16 * kWaves, kPt = kPos / 16;
  __shared__ __align__(16) uint8_t abuf[2][kPos * kActLds];
  __shared__ __align__(16) uint8_t dump[64 * 16];
  __shared__ uint32_t arow_lds[kPos];
  __shared__ uint64_t tab[32];
  const uint32_t nrb = g.row_blocks;
  const uint32_t nch = g.shared_T ? (g.shared_T + kPos - 1) / kPos : *g.ntiles, n = nch * nrb;
  if (blockIdx.x >= n) return;
  const uint32_t L = xcd_logical(blockIdx.x, n);
  const uint32_t ch_i = L / nrb, rb = L % nrb;
  uint32_t start, count, e;
  if (g.shared_T) {
    start = kPos * ch_i;
    count = min(kPos, g.shared_T - start), e = 0;
  } else {
    const MoeTile tl = g.tiles[ch_i];
    start = tl.start, count = tl.count, e = tl.slot;
  }
  const uint32_t tid = tid_fresh();
  if (tid < 32) tab[tid] = kExp2Tab[tid];
  if (tid < kPos) {
    const uint32_t pos = start + tid;
    arow_lds[tid] = tid < count ? (g.perm ? g.perm[pos] / g.K : pos) : 0xffffffffu;
  }
  __syncthreads();
  const uint32_t row0 = rb * kRows + 16 * (uint32_t)__builtin_amdgcn_readfirstlane(wave_id()), lane = lane_id();
  const uint8_t *Mg = g.mat + (uint64_t)e * g.stride, *Mu = Mg + g.up_off;
  const uint32_t npt = (count + 15) / 16;  // 16-position tiles with positions
  Dma<kPos, kWaves> dma;
  dma.plan(arow_lds, U);
  const __amdgpu_buffer_rsrc_t act_r = uniform_rsrc(g.act);
  Q4kBuf wb;
  wb.init(Mg, Mu, U, row0, lane);
  const auto load_w = [&](Q4kRaw &raw, uint32_t m, uint32_t u) { wb.load_qs(m, raw, u), wb.load_meta(m, raw, u); };
  Q4kRaw rg, ru;
  load_w(rg, 0, 0);
  load_w(ru, 1, 0);
  dma.load_all(act_r, 0, &abuf[0][0], dump);
  __builtin_amdgcn_s_waitcnt(vm_wait(0));
  unit_barrier();
  float accg[kPt][4], accu[kPt][4];
#pragma unroll
  for (int pt = 0; pt < (int)kPt; pt++)
#pragma unroll
    for (int i = 0; i < 4; i++) accg[pt][i] = accu[pt][i] = 0.0f;
  // Unit u; kNext: unit u + 1 exists (its loads are issued here). Compile-time, so that the compiler's waits for the
  // weight registers count the loads issued after them exactly. buf (read) and nbuf (filled) are restrict pointers:
  // the compiler then knows the reads of buf need not wait for the global-to-LDS loads into nbuf.
  const auto unit = [&](uint32_t u, auto kNext) {
    const auto body = [&](const uint8_t *__restrict__ buf, uint8_t *__restrict__ nbuf) {
      constexpr bool next = decltype(kNext)::value;
      if constexpr (next) dma.load_all(act_r, u + 1, nbuf, dump);  // the buffer unit u - 1 read before the barrier
      const auto pass = [&](Q4kRaw &raw, uint32_t m, float (&acc)[kPt][4]) {
        Q4kA a;
        pin(raw);  // the decode starts after the previous barrier ...
        a.decode<true>(raw, lane);
        pin(a);  // ... and ends before the next unit's loads into the raw registers
        if constexpr (next) load_w(raw, m, u + 1);
#pragma unroll
        for (uint32_t pt = 0; pt < kPt; pt++) {
          if (pt < npt) {
            ActBP b;
            b.load(buf + (16 * pt + lane % 16) * kActLds, lane);
            float t[4];
            q4k_terms_p(a, b, t);
#pragma unroll
            for (int i = 0; i < 4; i++) acc[pt][i] = __fadd_rn(acc[pt][i], t[i]);
          }
        }
      };
      pass(rg, 0, accg);
      pass(ru, 1, accu);
      if constexpr (next) {  // (after the last unit only the epilogue follows, which reads no activations)
        __builtin_amdgcn_s_waitcnt(vm_wait(0));  // unit u + 1's loads (this wave's) ...
        unit_barrier();                          // ... and every wave's; buffer u % 2 is free for unit u + 2
      }
    };
    body(abuf[u & 1], abuf[(u + 1) & 1]);
  };
#pragma unroll 1
  for (uint32_t u = 0; u + 1 < U; u++) unit(u, std::true_type{});
  unit(U - 1, std::false_type{});
  // Lane l holds rows row0 + 4 (l / 16) + i of positions 16 pt + l % 16, gate and up alike.
  const uint32_t r4 = 4 * (lane / 16), c16 = lane % 16;
#pragma unroll
  for (uint32_t pt = 0; pt < kPt; pt++)
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const uint32_t m = 16 * pt + c16;
      if (m < count) g.out[(uint64_t)(start + m) * g.out_ld + row0 + r4 + i] = swiglu_one(accg[pt][i], accu[pt][i], g.limit, tab);
    }
}

// IQ3_S gate/up at three waves a SIMD, in pf_gate_up_q4k's form: gate's products before up's, the activations one
// unit ahead in two LDS buffers, plain barriers. A block's A operand is decoded from the raw words (grid lookups in
// LDS) just before its MFMAs, so only the raw words and one block's operand are live (144 registers); each block's
// dots times the row's odd block scale are added to the unit's integer sums in block order, then d ad isum as
// UnitIQ3_S::term, units added in sequence. The raw registers take the next unit's loads (buffer loads on scalar
// bases, Iq3sBuf) once the pass has read them. Against the earlier form (both matrices in one wave, 220 registers,
// two waves a SIMD, activations two units ahead): 367 -> 350 us a launch at config 5p; the buffer loads (in place
// of global loads, 168 registers and a reload from scratch a unit) 358 -> 329 us.
template <uint32_t kPos>
__global__ void __launch_bounds__(4 * kPos) __attribute__((amdgpu_waves_per_eu(3))) pf_gate_up_iq3s(PfGemm g) {
  const uint32_t U = g.U;
  constexpr uint32_t kWaves = kPos / 16, kRows = 16 * kWaves, kPt = kPos / 16;
  __shared__ __align__(16) uint8_t abuf[2][kPos * kActLds];
  __shared__ __align__(16) uint8_t dump[64 * 16];
  __shared__ uint32_t arow_lds[kPos];
  __shared__ uint64_t tab[32];
  __shared__ uint32_t grid_lds[512];
  const uint32_t nrb = g.row_blocks;
  const uint32_t nch = g.shared_T ? (g.shared_T + kPos - 1) / kPos : *g.ntiles, n = nch * nrb;
  if (blockIdx.x >= n) return;
  const uint32_t L = xcd_logical(blockIdx.x, n);
  const uint32_t ch_i = L / nrb, rb = L % nrb;
  uint32_t start, count, e;
  if (g.shared_T) {
    start = kPos * ch_i;
    count = min(kPos, g.shared_T - start), e = 0;
  } else {
    const MoeTile tl = g.tiles[ch_i];
    start = tl.start, count = tl.count, e = tl.slot;
  }
  const uint32_t tid = tid_fresh();
  if (tid < 32) tab[tid] = kExp2Tab[tid];
  for (uint32_t i = tid; i < 512; i += 64 * kWaves) grid_lds[i] = kIq3sGridPf[i];
  if (tid < kPos) {
    const uint32_t pos = start + tid;
    arow_lds[tid] = tid < count ? (g.perm ? g.perm[pos] / g.K : pos) : 0xffffffffu;
  }
  __syncthreads();
  const uint32_t row0 = rb * kRows + 16 * (uint32_t)__builtin_amdgcn_readfirstlane(wave_id()), lane = lane_id();
  const uint8_t *Mg = g.mat + (uint64_t)e * g.stride, *Mu = Mg + g.up_off;
  const uint32_t npt = (count + 15) / 16;  // 16-position tiles with positions
  Dma<kPos, kWaves> dma;
  dma.plan(arow_lds, U);
  const __amdgpu_buffer_rsrc_t act_r = uniform_rsrc(g.act);
  Iq3sBuf wb;  // buffer loads on scalar bases (168 registers and a reload from scratch a unit with global loads)
  wb.init(Mg, Mu, U, row0, lane);
  const auto load_w = [&](Iq3sRaw &raw, uint32_t m, uint32_t u) { wb.load(m, raw, u); };
  Iq3sRaw rg, ru;
  load_w(rg, 0, 0);
  load_w(ru, 1, 0);
  dma.load_all(act_r, 0, &abuf[0][0], dump);
  __builtin_amdgcn_s_waitcnt(vm_wait(0));
  unit_barrier();
  float accg[kPt][4], accu[kPt][4];
#pragma unroll
  for (int pt = 0; pt < (int)kPt; pt++)
#pragma unroll
    for (int i = 0; i < 4; i++) accg[pt][i] = accu[pt][i] = 0.0f;
  // Unit u; kNext: unit u + 1 exists (its loads are issued here). Compile-time, so that the compiler's waits for the
  // weight registers count the loads issued after them exactly. buf (read) and nbuf (filled) are restrict pointers:
  // the compiler then knows the reads of buf need not wait for the global-to-LDS loads into nbuf.
  const auto unit = [&](uint32_t u, auto kNext) {
    const auto body = [&](const uint8_t *__restrict__ buf, uint8_t *__restrict__ nbuf) {
      constexpr bool next = decltype(kNext)::value;
      if constexpr (next) dma.load_all(act_r, u + 1, nbuf, dump);  // the buffer unit u - 1 read before the barrier
      const auto pass = [&](Iq3sRaw &raw, uint32_t m, float (&acc)[kPt][4]) {
        // Block by block: the block's A operand decoded (grid lookups), its dots for every position tile times the
        // row's odd block scale, added to the unit's integer sums in block order; then d ad isum.
        pin(raw);
        int is[kPt][4];
#pragma unroll
        for (int pt = 0; pt < (int)kPt; pt++)
#pragma unroll
          for (int i = 0; i < 4; i++) is[pt][i] = 0;
#pragma unroll
        for (uint32_t ib = 0; ib < 8; ib++) {
          const long aw = raw.a_block(ib, lane, grid_lds);
          const uint32_t bofs = mfma_code_off(4 * ib + lane / 16);
          int ls[4];
#pragma unroll
          for (uint32_t i = 0; i < 4; i++) ls[i] = raw.ls(i, ib);
#pragma unroll
          for (uint32_t pt = 0; pt < kPt; pt++) {
            if (pt < npt) {
              const long bw = *(const long *)(buf + (16 * pt + lane % 16) * kActLds + bofs);
              const v4i_t d = __builtin_amdgcn_mfma_i32_16x16x32_i8(aw, bw, v4i_t{0, 0, 0, 0}, 0, 0, 0);
#pragma unroll
              for (int i = 0; i < 4; i++) is[pt][i] += __mul24(ls[i], d[i]);
            }
          }
        }
        float dd[4];
#pragma unroll
        for (int i = 0; i < 4; i++) dd[i] = h2f((uint16_t)raw.dh[i]);
        pin(raw);
        if constexpr (next) load_w(raw, m, u + 1);  // the raw registers are free once the pass has read them
#pragma unroll
        for (uint32_t pt = 0; pt < kPt; pt++) {
          if (pt < npt) {
            const float ad = *(const float *)(buf + (16 * pt + lane % 16) * kActLds + kActScales);
#pragma unroll
            for (int i = 0; i < 4; i++) acc[pt][i] = __fadd_rn(acc[pt][i], __fmul_rn(__fmul_rn(dd[i], ad), (float)is[pt][i]));
          }
        }
      };
      pass(rg, 0, accg);
      pass(ru, 1, accu);
      if constexpr (next) {  // (after the last unit only the epilogue follows, which reads no activations)
        __builtin_amdgcn_s_waitcnt(vm_wait(0));  // unit u + 1's loads (this wave's) ...
        unit_barrier();                          // ... and every wave's; buffer u % 2 is free for unit u + 2
      }
    };
    body(abuf[u & 1], abuf[(u + 1) & 1]);
  };
#pragma unroll 1
  for (uint32_t u = 0; u + 1 < U; u++) unit(u, std::true_type{});
  unit(U - 1, std::false_type{});
  // Lane l holds rows row0 + 4 (l / 16) + i of positions 16 pt + l % 16, gate and up alike.
  const uint32_t r4 = 4 * (lane / 16), c16 = lane % 16;
#pragma unroll
  for (uint32_t pt = 0; pt < kPt; pt++)
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const uint32_t m = 16 * pt + c16;
      if (m < count) g.out[(uint64_t)(start + m) * g.out_ld + row0 + r4 + i] = swiglu_one(accg[pt][i], accu[pt][i], g.limit, tab);
    }
}

// Positions a gate/up work-group takes for a weight type (the kernel's kPos).
constexpr uint32_t gu_pos(uint32_t) { return MOE_TILE; }
// The gate/up types that run on pf_gate_up_q4k / pf_gate_up_iq3s (gate and up of a row in one wave); the others on
// pf_gemm16.
constexpr bool gu_fused(uint32_t type) { return type == QT_Q4_K || type == QT_IQ3_S; }

// ---------------------------------------------------------------------------------------------------------------
// Combine: y[t][r] = sum_k w[t][k] y_asg[inv[t K + k]][r] in rank order (ranks with a negative id skipped), then
// + gs[t] y_sh[t][r]; four rows a thread. The ranks go in batches of eight whose row loads are all issued before the
// first is added (rows of skipped ranks are not loaded and add nothing).

// With the token uniform a work-group, batches of 4, 8, 10 and 16 measured the same (34.2-34.5 us at config 4); with
// the token per thread, 12 and 16 measured 44 and 51 against 8's 38 us.
constexpr uint32_t kCombBatch = 8;

__global__ void __launch_bounds__(kPfWG) pf_combine(const float *y_asg, const uint32_t *inv, const int32_t *ids,
                                                    const float *w, uint32_t K, const float *y_sh, const float *gs,
                                                    uint32_t T, uint32_t H, float *y) {
  // Token blockIdx.y, uniform a work-group, so its ids, weights and positions are scalar loads (a token a thread,
  // with them as vector loads, measured 38 against 34 us at config 4); float4 column blockIdx.x kPfWG + tid.
  const uint32_t H4 = H / 4, t = blockIdx.y, r4 = blockIdx.x * kPfWG + threadIdx.x;
  if (t >= T || r4 >= H4) return;
  float4 acc = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
  for (uint32_t k0 = 0; k0 < K; k0 += kCombBatch) {
    float wk[kCombBatch];
    float4 v[kCombBatch];
    uint32_t used = 0;
#pragma unroll
    for (uint32_t j = 0; j < kCombBatch; j++) {
      const uint64_t a = (uint64_t)t * K + k0 + j;
      const bool use = k0 + j < K && ids[a] >= 0;  // a pre-routed token's unused rank: skipped
      used |= (uint32_t)use << j;
      wk[j] = use ? w[a] : 0.0f;
      v[j] = use ? ((const float4 *)(y_asg + (uint64_t)inv[a] * H))[r4] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    }
#pragma unroll
    for (uint32_t j = 0; j < kCombBatch; j++) {
      if (!(used >> j & 1u)) continue;
      acc.x = __fadd_rn(acc.x, __fmul_rn(wk[j], v[j].x)), acc.y = __fadd_rn(acc.y, __fmul_rn(wk[j], v[j].y));
      acc.z = __fadd_rn(acc.z, __fmul_rn(wk[j], v[j].z)), acc.w = __fadd_rn(acc.w, __fmul_rn(wk[j], v[j].w));
    }
  }
  if (y_sh) {
    const float g = gs[t];
    const float4 v = ((const float4 *)(y_sh + (uint64_t)t * H))[r4];
    acc.x = __fadd_rn(acc.x, __fmul_rn(g, v.x)), acc.y = __fadd_rn(acc.y, __fmul_rn(g, v.y));
    acc.z = __fadd_rn(acc.z, __fmul_rn(g, v.z)), acc.w = __fadd_rn(acc.w, __fmul_rn(g, v.w));
  }
  ((float4 *)(y + (uint64_t)t * H))[r4] = acc;
}

// ---------------------------------------------------------------------------------------------------------------
// Host side.

// pf_combine's grid: (H / 4 columns in work-groups of kPfWG) x T tokens.
inline dim3 comb_grid(uint32_t T, uint32_t H) { return dim3((H / 4 + kPfWG - 1) / kPfWG, T); }

// Row blocks a Q4_K down work-group walks, a power of two (config 4's routed down: 1 120, 2 107, 4 103, 8 105 us).
constexpr uint32_t kSharedGuLds = 16384;  // dynamic LDS reserved by the shared Q8_0 gate/up launch (not used)
constexpr uint32_t kDownSpan = 4;
constexpr uint32_t kDownMinGroups = 512;  // work-groups a walking down grid keeps (two a CU)

template <bool kGU>
void launch_gemm(uint32_t type, uint32_t U, dim3 grid, const PfGemm &g, hipStream_t s) {
  PfGemm q = g;
  q.U = U;
  if (kGU && gu_fused(type)) {  // gate and up in one wave: grid.x tiles x grid.y row blocks of gu_pos rows
    q.row_blocks = grid.y;
    const dim3 g2(grid.x * q.row_blocks), wg(4 * MOE_TILE);
    if (type == QT_Q4_K)
      pf_gate_up_q4k<MOE_TILE><<<g2, wg, 0, s>>>(q);
    else
      pf_gate_up_iq3s<MOE_TILE><<<g2, wg, 0, s>>>(q);
    return;
  }
  // The 16 x 16 MFMA kernel: 32 gate + 32 up rows, or 64 down rows, a work-group; a 1-D XCD-aware grid.
  q.row_blocks = grid.y * gemm_rows<kGU>() / (kGU ? 32 : 64);
  q.rb_span = 1;
  if (!kGU && type == QT_Q4_K && U <= 2) {  // down: the activations of both units stay in LDS while the work-group walks row blocks
    // Fewer row blocks a work-group where the grid would leave fewer than two work-groups a CU (the shared
    // expert's 32 tiles at 2048 tokens: span 2 15.7 against span 4 18.0 us).
    q.rb_span = kDownSpan;
    while (q.rb_span > 1 && (q.row_blocks % q.rb_span || grid.x * (q.row_blocks / q.rb_span) < kDownMinGroups))
      q.rb_span /= 2;
    q.row_blocks /= q.rb_span;
  }
  const dim3 g2(grid.x * q.row_blocks);
  if (kGU && q.shared_T && type == QT_Q8_0) {
    // The shared expert's Q8_0 gate/up runs beside the router and top-k on the side stream; at three work-groups a
    // CU it takes every register of the CUs it holds. kSharedGuLds of LDS it does not use caps it at two, leaving a
    // wave a SIMD to the top-k (config 5p: top-k 46 -> 33 us, this launch 51 -> 71, a step 52.8 -> 52.5 ms).
    pf_gemm16<QT_Q8_0, kGU><<<g2, kPfWG, kSharedGuLds, s>>>(q);
    return;
  }
  if (type == QT_Q4_K)
    pf_gemm16<QT_Q4_K, kGU><<<g2, kPfWG, 0, s>>>(q);
  else if (type == QT_IQ3_S)
    pf_gemm16<QT_IQ3_S, kGU><<<g2, kPfWG, 0, s>>>(q);
  else if (type == QT_IQ4_NL)
    pf_gemm16<QT_IQ4_NL, kGU><<<g2, kPfWG, 0, s>>>(q);
  else if (type == QT_IQ3_XXS)
    pf_gemm16<QT_IQ3_XXS, kGU><<<g2, kPfWG, 0, s>>>(q);
  else if (type == QT_IQ2_S)
    pf_gemm16<QT_IQ2_S, kGU><<<g2, kPfWG, 0, s>>>(q);
  else if (type == QT_Q2_0)
    pf_gemm16<QT_Q2_0, kGU><<<g2, kPfWG, 0, s>>>(q);
  else if (type == QT_IQ4_XS)
    pf_gemm16<QT_IQ4_XS, kGU><<<g2, kPfWG, 0, s>>>(q);
  else if (type == QT_Q5_K)
    pf_gemm16<QT_Q5_K, kGU><<<g2, kPfWG, 0, s>>>(q);
  else if (type == QT_Q6_K)
    pf_gemm16<QT_Q6_K, kGU><<<g2, kPfWG, 0, s>>>(q);
  else
    pf_gemm16<QT_Q8_0, kGU><<<g2, kPfWG, 0, s>>>(q);
}

struct HookScope {
  const PfHook &h;
  const char *name;
  hipStream_t s;
  HookScope(const PfHook &hk, const char *n, hipStream_t st) : h(hk), name(n), s(st) {
    if (h.fn) h.fn(h.ctx, name, 0, s);
  }
  ~HookScope() {
    if (h.fn) h.fn(h.ctx, name, 1, s);
  }
};

// Gate/up (SwiGLU into h) over nx tiles or chunks (at most; the kernel reads how many there are): Q4_K and IQ3_S on
// pf_gate_up_q4k / pf_gate_up_iq3s (gu_pos positions and rows of each a work-group), the other types on pf_gemm16
// (64-position tiles, 32 rows of gate and of up a work-group).
// Explicit instantiations: with only the implicit ones, this compiler's host pass emits the launch stub of the
// first instantiation of a kernel template whose body holds a lambda and silently drops the later ones (and with
// them launch_gemm<false>), which then fail at load time as undefined symbols.
template __global__ void pf_gate_up_q4k<MOE_TILE>(PfGemm);
template __global__ void pf_gate_up_iq3s<MOE_TILE>(PfGemm);
#define C0VEN_PF_GEMM16(T)                          \
  template __global__ void pf_gemm16<T, true>(PfGemm); \
  template __global__ void pf_gemm16<T, false>(PfGemm);
C0VEN_PF_GEMM16(QT_Q4_K)
C0VEN_PF_GEMM16(QT_IQ3_S)
C0VEN_PF_GEMM16(QT_Q8_0)
C0VEN_PF_GEMM16(QT_IQ4_NL)
C0VEN_PF_GEMM16(QT_Q2_0)
C0VEN_PF_GEMM16(QT_IQ3_XXS)
C0VEN_PF_GEMM16(QT_IQ2_S)
C0VEN_PF_GEMM16(QT_IQ4_XS)
C0VEN_PF_GEMM16(QT_Q5_K)
C0VEN_PF_GEMM16(QT_Q6_K)
#undef C0VEN_PF_GEMM16
template void launch_gemm<false>(uint32_t, uint32_t, dim3, const PfGemm &, hipStream_t);
template void launch_gemm<true>(uint32_t, uint32_t, dim3, const PfGemm &, hipStream_t);

void launch_gate_up(uint32_t type, const PfGemm &q, uint32_t T, uint32_t F, uint32_t Ug, uint32_t nx, hipStream_t s) {
  (void)T;
  const uint32_t ny = gu_fused(type) ? F / gu_pos(type) : F / gemm_rows<true>();
  launch_gemm<true>(type, Ug, dim3(nx, ny), q, s);
}

// The routed experts of a forward whose ids and w (T x K, ids < 0 for no assignment) are in b: dispatch, gate/up,
// h quantiser, down (y per assignment in b.y_asg). masks_built: b.masks already hold the ids' window masks (pf_topk).
hipError_t routed_experts(const PfShape &S, const PfLayer &L, const PfBufs &b, hipStream_t st, const PfHook &hook,
                          bool masks_built) {
  const uint32_t H = S.H, F = S.F, E = S.E, K = S.K, T = S.T, Ug = units_of(H), Ud = units_of(F);
  const uint32_t hr = quant_vec_dot_type(S.down_type);
  const uint32_t halfwaves = kPfWG / 32;
  const uint32_t mt = pf_max_tiles(T, K, E);
  {
    HookScope k(hook, "pf_dispatch", st);
    const uint32_t nwin = pf_windows(T);
    if (!masks_built) pf_masks<<<nwin, kDispWG, 0, st>>>(b.ids, T, K, E, b.masks);
    pf_place<<<nwin, kDispWG, 0, st>>>(b.ids, T, K, E, nwin, b.masks, b.tiles, b.ntiles, b.perm, b.inv);
  }
  {
    HookScope k(hook, "pf_gate_up", st);
    PfGemm g{};
    g.tiles = b.tiles, g.ntiles = b.ntiles, g.perm = b.perm, g.K = K, g.act = b.act_r, g.act_by_pos = 0;
    g.mat = L.experts, g.stride = L.ex_bytes, g.up_off = L.ex_up_off, g.out = b.h, g.out_ld = F;
    g.codebooks = L.codebooks;
    g.limit = S.swiglu_limit;
    launch_gate_up(S.gate_type, g, T, F, Ug, mt, st);
  }
  {
    HookScope k(hook, "pf_quant_h", st);
    pf_quant_rows<<<(T * K * Ud + halfwaves - 1) / halfwaves, kPfWG, 0, st>>>(b.h, F, T * K, Ud, hr, b.hact, 0,
                                                                              nullptr);
  }
  {
    HookScope k(hook, "pf_down", st);
    PfGemm g{};
    g.tiles = b.tiles, g.ntiles = b.ntiles, g.K = K, g.act = b.hact, g.act_by_pos = 1;
    g.mat = L.experts + L.ex_down_off, g.stride = L.ex_bytes, g.out = b.y_asg, g.out_ld = H;
    g.codebooks = L.codebooks;
    launch_gemm<false>(S.down_type, Ud, dim3(mt, H / gemm_rows<false>()), g, st);
  }
  return hipGetLastError();
}

}  // namespace

hipError_t prefill_forward(const PfShape &S, const PfLayer &L, const PfBufs &b, const float *x, float *y, hipStream_t st,
                     const PfHook &hook) {
  const uint32_t H = S.H, F = S.F, E = S.E, K = S.K, T = S.T, Ug = units_of(H), Ud = units_of(F);
  const uint32_t xr = quant_vec_dot_type(S.gate_type);
  const uint32_t xs = S.has_shared ? quant_vec_dot_type(S.sh_gate_type) : xr;
  const uint32_t hs = quant_vec_dot_type(S.sh_down_type);
  const uint32_t halfwaves = kPfWG / 32;
  // The x quantiser: on the side stream with a shared expert (the router reads x itself; the routed launches wait for
  // it after the top-k), else first on the block's stream.
  const auto quant_x = [&](hipStream_t s) {
    HookScope k(hook, "pf_quant_x", s);
    pf_quant_rows<<<(T * Ug + halfwaves - 1) / halfwaves, kPfWG, 0, s>>>(x, H, T, Ug, xr, b.act_r, xs,
                                                                           b.act_s != b.act_r ? b.act_s : nullptr);
  };
  const uint32_t st_tiles = (T + MOE_TILE - 1) / MOE_TILE;
  if (!S.has_shared) quant_x(st);
  if (S.has_shared) {  // the shared expert needs no routing: its launches run beside the router on the side stream
    hipStream_t ss = b.side;
    if (hipEventRecord(b.fork, st) != hipSuccess || hipStreamWaitEvent(ss, b.fork, 0) != hipSuccess)
      return hipGetLastError();
    quant_x(ss);
    if (hipEventRecord(b.xq, ss) != hipSuccess) return hipGetLastError();
    if (S.sh_up_type == S.sh_gate_type) {
      {
        HookScope k(hook, "pf_gate_up_shared", ss);
        PfGemm q{};
        q.shared_T = T, q.K = K, q.act = b.act_s, q.act_by_pos = 0;
        q.mat = L.shared, q.stride = 0, q.up_off = L.sh_up_off, q.out = b.h_sh, q.out_ld = F;
        q.codebooks = L.codebooks;
        q.limit = S.swiglu_limit;
        launch_gate_up(S.sh_gate_type, q, T, F, Ug, (T + gu_pos(S.sh_gate_type) - 1) / gu_pos(S.sh_gate_type), ss);
      }
      {
        HookScope k(hook, "pf_quant_h_shared", ss);
        pf_quant_rows<<<(T * Ud + halfwaves - 1) / halfwaves, kPfWG, 0, ss>>>(b.h_sh, F, T, Ud, hs, b.hact_sh, 0,
                                                                              nullptr);
      }
    } else {  // gate and up of different types: two plain GEMMs (the reference's two matvecs), SwiGLU in the quantiser
      for (uint32_t m = 0; m < 2; m++) {
        HookScope k(hook, m ? "pf_up_shared" : "pf_gate_shared", ss);
        PfGemm q{};
        q.shared_T = T, q.K = K, q.act = b.act_s, q.act_by_pos = 0;
        q.mat = L.shared + (m ? L.sh_up_off : 0), q.stride = 0, q.out = m ? b.h_sh_up : b.h_sh, q.out_ld = F;
        q.codebooks = L.codebooks;
        launch_gemm<false>(m ? S.sh_up_type : S.sh_gate_type, Ug, dim3(st_tiles, F / gemm_rows<false>()), q, ss);
      }
      HookScope k(hook, "pf_quant_h_shared", ss);
      pf_quant_swiglu<<<(T * Ud + halfwaves - 1) / halfwaves, kPfWG, 0, ss>>>(b.h_sh, b.h_sh_up, F, T, Ud,
                                                                              S.swiglu_limit, hs, b.hact_sh);
    }
    {
      HookScope k(hook, "pf_down_shared", ss);
      PfGemm q{};
      q.shared_T = T, q.K = K, q.act = b.hact_sh, q.act_by_pos = 1;
      q.mat = L.shared + L.sh_down_off, q.stride = 0, q.out = b.y_sh, q.out_ld = H;
      q.codebooks = L.codebooks;
      launch_gemm<false>(S.sh_down_type, Ud, dim3(st_tiles, H / gemm_rows<false>()), q, ss);
    }
    if (hipEventRecord(b.join, ss) != hipSuccess) return hipGetLastError();
  }
  if (S.exact_router) {
    {
      HookScope k(hook, "pf_router", st);
      pf_router<<<dim3((T + 63) / 64, (E + 63) / 64 + 1), kPfWG, 0, st>>>(x, T, L.router, L.bias, E, H, b.logits,
                                                                         b.masks);
    }
    {
      HookScope k(hook, "pf_topk", st);
      pf_topk<<<(T + 3) / 4, kPfWG, 0, st>>>(b.logits, T, E, K, b.ids, b.w, S.has_shared ? b.gs : nullptr, b.masks);
    }
  } else {
    {
      HookScope k(hook, "pf_xprep", st);
      pf_xprep<<<(T + 3) / 4, kPfWG, 0, st>>>(x, T, H, E, b.xb, b.xt, b.xn, b.xlsb, b.masks, L.router + (uint64_t)E * H,
                                              b.logits, S.has_shared ? b.gs : nullptr);
    }
    {
      HookScope k(hook, "pf_router", st);
      constexpr uint32_t kS = 2, kTile = 16 * kS;
      const uint32_t n = ((E + kTile - 1) / kTile) * ((T + kTile - 1) / kTile);
      pf_router_bf16<kS><<<n, kPfWG, 0, st>>>(L.router_t, b.xt, T, E, H, L.bias, b.logits);
    }
    {
      HookScope k(hook, "pf_topk", st);
      // 1.01 n 2^-23, n = 31 + H / 128 + 3 roundings a product may meet (see pf_router_bf16).
      const float gamma = (float)(1.01 * (31 + H / 128 + 3) * 0x1p-23);
      pf_topk_cert<<<(T + 3) / 4, kPfWG, 0, st>>>(b.logits, L.router, L.rlsb, b.xb, b.xn, b.xlsb, T, E, H, K, L.bias,
                                                  gamma * L.rmax * 1.0001f, L.bias_max, b.ids, b.w,
                                                  b.masks, b.cnt_exact);
    }
  }
  if (S.has_shared && hipStreamWaitEvent(st, b.xq, 0) != hipSuccess) return hipGetLastError();
  const hipError_t e = routed_experts(S, L, b, st, hook, true);
  if (e != hipSuccess) return e;
  if (S.has_shared && hipStreamWaitEvent(st, b.join, 0) != hipSuccess) return hipGetLastError();
  {
    HookScope k(hook, "pf_combine", st);
    pf_combine<<<comb_grid(T, H), kPfWG, 0, st>>>(b.y_asg, b.inv, b.ids, b.w, K,
                                                                        S.has_shared ? b.y_sh : nullptr, b.gs, T, H, y);
  }
  return hipGetLastError();
}

hipError_t prefill_jobs(const PfShape &S, const PfLayer &L, const PfBufs &b, const float *x, float *y, hipStream_t st,
                        const PfHook &hook) {
  const uint32_t H = S.H, K = S.K, T = S.T, Ug = units_of(H);
  const uint32_t halfwaves = kPfWG / 32;
  {
    HookScope k(hook, "pf_quant_x", st);
    pf_quant_rows<<<(T * Ug + halfwaves - 1) / halfwaves, kPfWG, 0, st>>>(x, H, T, Ug, quant_vec_dot_type(S.gate_type),
                                                                            b.act_r, 0, nullptr);
  }
  const hipError_t e = routed_experts(S, L, b, st, hook, false);
  if (e != hipSuccess) return e;
  {
    HookScope k(hook, "pf_combine", st);
    pf_combine<<<comb_grid(T, H), kPfWG, 0, st>>>(b.y_asg, b.inv, b.ids, b.w, K, nullptr, nullptr,
                                                                        T, H, y);
  }
  return hipGetLastError();
}

}  // namespace c0ven
