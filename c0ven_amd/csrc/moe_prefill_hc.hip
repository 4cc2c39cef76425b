// The hyper-connection mix before the prefill block and the combine after it (docs/spec/MODEL_LAYER.md 1.1-1.2; the
// reference's prompt path runs p_hc_mix and p_hc_combine around the block, core/models/qwen4exp/prompt.cpp:478-504).
//
// The results are the decode path's, bit for bit (and the oracle's, orc_hc_pre / orc_hc_post): the norms, silu,
// sigmoid and mix steps are the same fp32 operations; the two bf16 products (W_down and W_inject against n, W_up
// against l) are sums of exact products that the decode kernel adds in fp64 in a fixed order and rounds to fp32 once.
// Here they run on the fp64 matrix cores (v_mfma_f64_16x16x4f64) in another order, with a bound on the difference:
// each sum path has at most n_mine roundings here and n_ref in the fixed order, so the two fp64 values are within
// (n_mine + n_ref) 2^-53 sum|p| <= (n_mine + n_ref) 2^-53 ||w||_2 ||x||_2 of each other (Cauchy-Schwarz on the bf16
// values). Where the fp32 rounding of every value in that interval is the same, it is the fixed order's rounding; and
// where the products' bits span fewer than 53 (the least lsb of the row's and of the token's values against the
// Cauchy-Schwarz bound on sum|p|), both sums are exact, whatever their order (ties of fp32 rounding are common for
// W_up's short sums, and this settles them).
// Otherwise the sum is recomputed in the fixed order, one wave an open sum, from a list, in a kernel of its own:
// W_up's a k-order chain of at most 512 terms, W_down's and W_inject's the decode kernel's 512-value-chunk tree.
#include <hip/hip_runtime.h>

#include "device_math.h"
#include "prefill_hc.h"

namespace c0ven {
namespace {

typedef double v4d_t __attribute__((ext_vector_type(4)));

constexpr uint32_t kHcWG = 256;
constexpr uint32_t kHcStreams4 = 4;
constexpr uint32_t kGroupK = 128;  // values a matrix-core chain sums before its sum joins the fp64 total

__device__ __forceinline__ uint32_t lane_of() { return threadIdx.x & 63u; }

// The lsb exponent of a bf16 value's bits (2^(e - 134) for exponent field e, 2^-133 for a subnormal); a large value
// for zero, which adds no bits to a sum.
__device__ __forceinline__ int bf16_lsb_of(float v) {
  const uint32_t u = __float_as_uint(v), e = (u >> 23) & 0xffu;
  return (u & 0x7fff0000u) == 0u ? (1 << 20) : (e == 0u ? -133 : (int)e - 134);
}

__device__ __forceinline__ double bf16_lo(uint32_t w) { return (double)__uint_as_float(w << 16); }
__device__ __forceinline__ double bf16_hi(uint32_t w) { return (double)__uint_as_float(w & 0xffff0000u); }

// A double summed over the work-group (256) in a fixed order: each wave by halving exchanges, then the four waves.
__device__ __forceinline__ double wg_sum(double v, double *red) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = __dadd_rn(v, __shfl_xor(v, o, 64));
  __syncthreads();
  if (lane_of() == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  const double s = __dadd_rn(__dadd_rn(red[0], red[1]), __dadd_rn(red[2], red[3]));
  __syncthreads();
  return s;
}

__device__ __forceinline__ int wg_min(int v, int *red) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = min(v, __shfl_xor(v, o, 64));
  __syncthreads();
  if (lane_of() == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  const int m = min(min(red[0], red[1]), min(red[2], red[3]));
  __syncthreads();
  return m;
}

// Token t (one work-group): each stream as RMSNorm(R_s) gamma_s, the decode kernel's hc_norm_item arithmetic (each
// thread's squares in order, then wg_sum; mean rounded to fp32; 1 / sqrtf(mean + 1e-6)): the stream's scale into sc
// (pf_hc_mix forms n again from R, the scale and gamma), bf16(n) into nb, and the 2-norm (rounded up) and least lsb
// exponent of bf16(n). Work-group 0 clears the open lists' counts.
__global__ void __launch_bounds__(kHcWG) pf_hc_norm(const float *R, const float *gamma, uint32_t H, float *sc,
                                                    uint16_t *nb, double *nn, int *nlsb, uint32_t *cnt) {
  __shared__ double red[4];
  __shared__ int redi[4];
  int lsb = 1 << 20;
  const uint32_t t = blockIdx.x;
  if (t == 0 && threadIdx.x < 2) cnt[threadIdx.x] = 0u;
  double sq = 0.0;
  for (uint32_t s = 0; s < kHcStreams4; s++) {
    const float *r = R + ((uint64_t)t * kHcStreams4 + s) * H;
    double ss = 0.0;
    for (uint32_t i = threadIdx.x; i < H; i += kHcWG) ss = __dadd_rn(ss, (double)__fmul_rn(r[i], r[i]));
    ss = wg_sum(ss, red);
    const float mean = (float)(ss / (double)H);
    const float scale = __fdiv_rn(1.0f, sqrtf(__fadd_rn(mean, 1e-6f)));
    if (threadIdx.x == 0) sc[t * kHcStreams4 + s] = scale;
    uint16_t *ob = nb + ((uint64_t)t * kHcStreams4 + s) * H;
    for (uint32_t i = threadIdx.x; i < H; i += kHcWG) {
      const float v = __fmul_rn(__fmul_rn(r[i], scale), gamma[s * H + i]);
      const float bv = round_bf16(v);
      ob[i] = (uint16_t)(__float_as_uint(bv) >> 16);
      const double b = (double)bv;
      sq = __builtin_fma(b, b, sq);
      lsb = min(lsb, bf16_lsb_of(bv));
    }
  }
  sq = wg_sum(sq, red);
  lsb = wg_min(lsb, redi);
  if (threadIdx.x == 0) nn[t] = sqrt(sq) * (1.0 + 0x1p-30), nlsb[t] = lsb;
}

// Whether an fp64 sum v of a row's and a token's bf16 products rounds to fp32 as the fixed order's does. Exact: every
// product is a multiple of 2^(lr + lt) and sum|p| <= rn tn < 2^(lr + lt + 53), so every partial sum of any order is
// representable and both orders give the exact sum. Otherwise bounded: the two fp64 values are within bnd, and every
// value in [v - bnd, v + bnd] rounds to the same fp32.
__device__ __forceinline__ bool certain(double v, double rn, double tn, int lr, int lt, double bound_k) {
  if (!__builtin_isfinite(v)) return false;
  const double m = rn * tn;
  if (lr + lt < 900 && m < ldexp(1.0, lr + lt + 53)) return true;
  const double bnd = bound_k * m;
  const float f = (float)v;
  return (float)(v - bnd) == f && (float)(v + bnd) == f;
}

// C = A B^T on the fp64 matrix cores, both bf16: rows of A (M of them: A0's first M0, then A1's), tokens of B (N rows
// of K), K values. A work-group takes 64 rows x 64 tokens over the K range of its split
// (blockIdx.y), wave w rows 32 (w & 1) .. and tokens 32 (w >> 1) .., as 2 x 2 tiles of 16 x 16. Lane l (g = l / 16)
// holds A[row l % 16][k + 4 g + m] and B[token l % 16][k + 4 g + m] for MFMA step m of a 16-value chunk: both operands
// take the same k in the same place, so each step adds 64 of the row-token products (the order of a sum is free
// here: the bound covers any). Each kGroupK values' chain starts from zero and is added to an fp64 total.
// kUp: one split; the sums are certified here (row norms rn, token norms tn) and written as fp32 to out32 (N x M), an
// open one's (token, row) to the list open (pf_hc_up_fix writes it). Otherwise the fp64 totals go to part
// (split x N x M).
template <bool kUp>
__global__ void __launch_bounds__(kHcWG) pf_hc_gemm(const uint16_t *A0, uint32_t M0, const uint16_t *A1, uint32_t M,
                                                    uint32_t K, const uint16_t *B, uint32_t N, uint32_t ksplit,
                                                    double *part, float *out32, const double *rn, const double *tn,
                                                    const int *rl, const int *tl, double bound_k, uint32_t *open,
                                                    uint32_t *cnt) {
  const uint32_t nmt = (M + 63) / 64, mt = blockIdx.x % nmt, nt = blockIdx.x / nmt, split = blockIdx.y;
  const uint32_t lane = lane_of(), w = threadIdx.x >> 6, g = lane / 16, c16 = lane % 16;
  const uint32_t m0 = 64 * mt + 32 * (w & 1), n0 = 64 * nt + 32 * (w >> 1);
  // 16 x 16 tiles wholly past the rows or the tokens (the down GEMM's last row tile holds 4 of W_inject's rows) are
  // skipped: a wave with none returns (the kernel has no barrier), the others skip the MFMAs of theirs.
  if (m0 >= M || n0 >= N) return;
  const bool live_i1 = m0 + 16 < M, live_j1 = n0 + 16 < N;
  const uint16_t *ar[2];
  const uint16_t *br[2];
#pragma unroll
  for (int f = 0; f < 2; f++) {
    const uint32_t row = min(m0 + 16 * f + c16, M - 1), tok = min(n0 + 16 * f + c16, N - 1);
    ar[f] = row < M0 ? A0 + (uint64_t)row * K : A1 + (uint64_t)(row - M0) * K;
    br[f] = B + (uint64_t)tok * K;
  }
  const uint32_t kb = split * ksplit, ke = min(K, kb + ksplit);
  v4d_t tot[2][2];
#pragma unroll
  for (int i = 0; i < 2; i++)
#pragma unroll
    for (int j = 0; j < 2; j++) tot[i][j] = v4d_t{0.0, 0.0, 0.0, 0.0};
  for (uint32_t kg = kb; kg < ke; kg += kGroupK) {
    v4d_t acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
      for (int j = 0; j < 2; j++) acc[i][j] = v4d_t{0.0, 0.0, 0.0, 0.0};
    const uint32_t kge = min(ke, kg + kGroupK);
#pragma unroll 2
    for (uint32_t kc = kg; kc < kge; kc += 16) {
      const uint32_t k = kc + 4 * g;
      const bool ok = k < kge;  // (K is a multiple of 4: a lane's four values are all in or all out)
      uint2 a[2], b[2];
#pragma unroll
      for (int f = 0; f < 2; f++) {
        a[f] = ok ? *(const uint2 *)(ar[f] + k) : make_uint2(0u, 0u);
        b[f] = ok ? *(const uint2 *)(br[f] + k) : make_uint2(0u, 0u);
      }
      double ad[2][4], bd[2][4];
#pragma unroll
      for (int f = 0; f < 2; f++) {
        ad[f][0] = bf16_lo(a[f].x), ad[f][1] = bf16_hi(a[f].x), ad[f][2] = bf16_lo(a[f].y), ad[f][3] = bf16_hi(a[f].y);
        bd[f][0] = bf16_lo(b[f].x), bd[f][1] = bf16_hi(b[f].x), bd[f][2] = bf16_lo(b[f].y), bd[f][3] = bf16_hi(b[f].y);
      }
#pragma unroll
      for (int m = 0; m < 4; m++)
#pragma unroll
        for (int i = 0; i < 2; i++)
#pragma unroll
          for (int j = 0; j < 2; j++)
          if ((i == 0 || live_i1) && (j == 0 || live_j1))
            acc[i][j] = __builtin_amdgcn_mfma_f64_16x16x4f64(ad[i][m], bd[j][m], acc[i][j], 0, 0, 0);
    }
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
      for (int j = 0; j < 2; j++)
#pragma unroll
        for (int q = 0; q < 4; q++) tot[i][j][q] = __dadd_rn(tot[i][j][q], acc[i][j][q]);
  }
  // tot[i][j][q]: row m0 + 16 i + 4 q + g, token n0 + 16 j + c16 (the f64 form's result layout: element q of lane l
  // is row 4 q + l / 16).
#pragma unroll
  for (int i = 0; i < 2; i++)
#pragma unroll
    for (int j = 0; j < 2; j++)
#pragma unroll
      for (int q = 0; q < 4; q++) {
        const uint32_t row = m0 + 16 * i + 4 * q + g, tok = n0 + 16 * j + c16;
        if (row >= M || tok >= N) continue;
        const double v = tot[i][j][q];
        if constexpr (kUp) {
          if (certain(v, rn[row], tn[tok], rl[row], tl[tok], bound_k)) {
            out32[(uint64_t)tok * M + row] = (float)v;
          } else {  // open: pf_hc_up_fix writes it
            const uint32_t at = atomicAdd(cnt, 1u);
            open[2 * at] = tok, open[2 * at + 1] = row;
          }
        } else {
          part[((uint64_t)split * N + tok) * M + row] = v;
        }
      }
}

// Token t's down sums (rows < lr of W_down, then the 4 of W_inject): the splits added in order, certified against the
// fixed order (certain), rounded to fp32 into raw (T x (lr + 4)); an open one's (t, row) goes to the list (its
// raw entry is written by pf_hc_down_fix). force_open sends all.
__global__ void __launch_bounds__(kHcWG) pf_hc_down_fin(const double *part, uint32_t T, uint32_t M, uint32_t nsplit,
                                                        const double *rn, const double *tn, const int *rl,
                                                        const int *tl, double bound_k, bool force_open, float *raw,
                                                        uint32_t *open, uint32_t *cnt) {
  const uint32_t t = blockIdx.x;
  for (uint32_t row = threadIdx.x; row < M; row += kHcWG) {
    double v = 0.0;
    for (uint32_t s = 0; s < nsplit; s++) v = __dadd_rn(v, part[((uint64_t)s * T + t) * M + row]);
    if (!force_open && certain(v, rn[row], tn[t], rl[row], tl[t], bound_k)) {
      raw[(uint64_t)t * M + row] = (float)v;
    } else {
      const uint32_t at = atomicAdd(cnt, 1u);
      open[2 * at] = t, open[2 * at + 1] = row;
    }
  }
}

// The open down sums in the decode kernel's fixed order (bf16_dot for one row and one token, restated for one wave):
// 512-value chunks c; lane l's eight values 8 l .. 8 l + 7 a fused chain from zero; a lane row r (16 lanes) as
// ((P0 + P7) + (P3 + P4)) + ((P1 + P6) + (P2 + P5)), P_m = a_m + a_(15 - m); slot 4 (c mod 4) + r takes the chunks'
// sums in chunk order; the 16 slots added in order from zero. One wave an entry.
__global__ void __launch_bounds__(kHcWG) pf_hc_down_fix(const uint16_t *w_down, const uint16_t *w_inj, uint32_t lr,
                                                        uint32_t K, const uint16_t *nb, const uint32_t *open,
                                                        const uint32_t *cnt, float *raw) {
  const uint32_t lane = lane_of(), r = lane / 16, nw = gridDim.x * (kHcWG / 64), M = lr + kHcStreams4;
  for (uint32_t e = blockIdx.x * (kHcWG / 64) + (threadIdx.x >> 6); e < *cnt; e += nw) {
    const uint32_t t = open[2 * e], row = open[2 * e + 1];
    const uint16_t *wr = row < lr ? w_down + (uint64_t)row * K : w_inj + (uint64_t)(row - lr) * K;
    const uint16_t *xr = nb + (uint64_t)t * K;
    double slot[4] = {0.0, 0.0, 0.0, 0.0};  // slot 4 w + r, w = c mod 4 (lane 16 r holds its row's)
    for (uint32_t c = 0; c < K / 512; c++) {
      const uint32_t k0 = 512 * c + 8 * lane;
      const uint4 wq = *(const uint4 *)(wr + k0), xq = *(const uint4 *)(xr + k0);
      const uint32_t ww[4] = {wq.x, wq.y, wq.z, wq.w}, xw[4] = {xq.x, xq.y, xq.z, xq.w};
      double a = 0.0;
#pragma unroll
      for (int k = 0; k < 8; k++)
        a = __builtin_fma((k & 1) ? bf16_hi(ww[k / 2]) : bf16_lo(ww[k / 2]), (k & 1) ? bf16_hi(xw[k / 2]) : bf16_lo(xw[k / 2]), a);
      const double P = __dadd_rn(a, __shfl_xor(a, 15, 64));  // lanes m < 8 of a row: P_m
      double p[8];
#pragma unroll
      for (int j = 0; j < 8; j++) p[j] = __shfl(P, (int)(16 * r + j), 64);
      const double S = __dadd_rn(__dadd_rn(__dadd_rn(p[0], p[7]), __dadd_rn(p[3], p[4])),
                                 __dadd_rn(__dadd_rn(p[1], p[6]), __dadd_rn(p[2], p[5])));
#pragma unroll
      for (uint32_t q = 0; q < 4; q++)
        if ((c & 3u) == q) slot[q] = c < 4 ? S : __dadd_rn(slot[q], S);
    }
    double s = 0.0;
#pragma unroll
    for (uint32_t q = 0; q < 4; q++)
#pragma unroll
      for (uint32_t rr = 0; rr < 4; rr++) s = __dadd_rn(s, __shfl(slot[q], (int)(16 * rr), 64));
    if (lane == 0) raw[(uint64_t)t * M + row] = (float)s;
  }
}

// The open up sums in the fixed order: a k-order chain over the lr values of W_up's row against bf16(l) of the token,
// one fused step a term from zero. One wave an entry: the wave brings the row and l into its LDS, lane 0 runs the
// chain from there.
__global__ void __launch_bounds__(kHcWG) pf_hc_up_fix(const uint16_t *w_up, uint32_t lr, uint32_t M, const uint16_t *lb,
                                                      const uint32_t *open, const uint32_t *cnt, float *out32) {
  __shared__ __align__(16) float ws[kHcWG / 64][512], xs[kHcWG / 64][512];
  const uint32_t lane = lane_of(), wv = threadIdx.x >> 6, nw = gridDim.x * (kHcWG / 64);
  for (uint32_t e = blockIdx.x * (kHcWG / 64) + wv; e < *cnt; e += nw) {
    const uint32_t t = open[2 * e], row = open[2 * e + 1];
    const uint16_t *wr = w_up + (uint64_t)row * lr;
    const uint16_t *xr = lb + (uint64_t)t * lr;
    for (uint32_t k = lane; k < lr; k += 64) {
      ws[wv][k] = __uint_as_float((uint32_t)wr[k] << 16);
      xs[wv][k] = __uint_as_float((uint32_t)xr[k] << 16);
    }
    __builtin_amdgcn_s_waitcnt(0xc07f);
    __builtin_amdgcn_wave_barrier();
    if (lane == 0) {
      double c = 0.0;
      for (uint32_t k = 0; k < lr; k += 4) {
        const float4 w4 = *(const float4 *)&ws[wv][k], x4 = *(const float4 *)&xs[wv][k];
        c = __builtin_fma((double)w4.x, (double)x4.x, c);
        c = __builtin_fma((double)w4.y, (double)x4.y, c);
        c = __builtin_fma((double)w4.z, (double)x4.z, c);
        c = __builtin_fma((double)w4.w, (double)x4.w, c);
      }
      out32[(uint64_t)t * M + row] = (float)c;
    }
    __builtin_amdgcn_wave_barrier();
  }
}

// Token t: l = silu(v / 4) for W_down's rows (the quarter exact; z / (1 + e^-z)) as bf16 bits (the up GEMM's operand),
// the inject logits for W_inject's, and the 2-norm (rounded up) and least lsb exponent of bf16(l).
__global__ void __launch_bounds__(kHcWG) pf_hc_down_epi(const float *raw, uint32_t lr, uint16_t *lb, float *inj,
                                                        double *ln, int *llsb) {
  __shared__ uint64_t tab[32];
  __shared__ double red[4];
  __shared__ int redi[4];
  int lsb = 1 << 20;
  if (threadIdx.x < 32) tab[threadIdx.x] = kExp2Tab[threadIdx.x];
  __syncthreads();
  const uint32_t t = blockIdx.x, M = lr + kHcStreams4;
  double sq = 0.0;
  for (uint32_t j = threadIdx.x; j < M; j += kHcWG) {
    const float v = raw[(uint64_t)t * M + j];
    if (j < lr) {
      const float z = __fmul_rn(v, 0.25f);
      const float o = __fdiv_rn(z, __fadd_rn(1.0f, expf_libm(-z, tab)));
      const float bo = round_bf16(o);
      lb[(uint64_t)t * lr + j] = (uint16_t)(__float_as_uint(bo) >> 16);
      const double b = (double)bo;
      sq = __builtin_fma(b, b, sq);
      lsb = min(lsb, bf16_lsb_of(bo));
    } else {
      inj[(uint64_t)t * kHcStreams4 + j - lr] = v;
    }
  }
  sq = wg_sum(sq, red);
  lsb = wg_min(lsb, redi);
  if (threadIdx.x == 0) ln[t] = sqrt(sq) * (1.0 + 0x1p-30), llsb[t] = lsb;
}

// x[t][i] = (sum over s in order of n_s[i] sigma(a_s[i])) / 4 with n_s[i] = (R_s[i] sc_s) gamma_s[i] (pf_hc_norm's
// product), a thread two consecutive values (H is a multiple of 512, so a work-group's 512 values are one token's);
// every load issued before the first is used.
__global__ void __launch_bounds__(kHcWG) pf_hc_mix(const float *R, const float *gamma, const float *sc, const float *a,
                                                   uint32_t T, uint32_t H, float *x) {
  __shared__ uint64_t tab[32];
  if (threadIdx.x < 32) tab[threadIdx.x] = kExp2Tab[threadIdx.x];
  __syncthreads();
  const uint64_t e = ((uint64_t)blockIdx.x * kHcWG + threadIdx.x) * 2;
  if (e >= (uint64_t)T * H) return;
  const uint32_t t = (uint32_t)(e / H), i = (uint32_t)(e % H);
  float2 nv[kHcStreams4], av[kHcStreams4], gv[kHcStreams4];
  float scale[kHcStreams4];
#pragma unroll
  for (uint32_t s = 0; s < kHcStreams4; s++) {
    const uint64_t o = ((uint64_t)t * kHcStreams4 + s) * H + i;
    nv[s] = *(const float2 *)(R + o), av[s] = *(const float2 *)(a + o), gv[s] = *(const float2 *)(gamma + s * H + i);
    scale[s] = sc[t * kHcStreams4 + s];
  }
  float2 acc = make_float2(0.0f, 0.0f);
#pragma unroll
  for (uint32_t s = 0; s < kHcStreams4; s++) {
    nv[s].x = __fmul_rn(__fmul_rn(nv[s].x, scale[s]), gv[s].x);
    nv[s].y = __fmul_rn(__fmul_rn(nv[s].y, scale[s]), gv[s].y);
    acc.x = __fadd_rn(acc.x, __fmul_rn(nv[s].x, sigmoid_libm(av[s].x, tab)));
    acc.y = __fadd_rn(acc.y, __fmul_rn(nv[s].y, sigmoid_libm(av[s].y, tab)));
  }
  *(float2 *)(x + e) = make_float2(__fmul_rn(acc.x, 0.25f), __fmul_rn(acc.y, 0.25f));
}

// R_s[i] += 2 sigma(inject_s / 4) y[i], a thread two consecutive values of a token (a work-group's 512 values are one
// token's: H is a multiple of 512), the four stream weights worked out once a work-group.
__global__ void __launch_bounds__(kHcWG) pf_hc_post(float *R, const float *y, const float *inj, uint32_t T,
                                                    uint32_t H) {
  __shared__ uint64_t tab[32];
  __shared__ float ws[kHcStreams4];
  if (threadIdx.x < 32) tab[threadIdx.x] = kExp2Tab[threadIdx.x];
  __syncthreads();
  const uint64_t e0 = (uint64_t)blockIdx.x * kHcWG * 2, e = e0 + 2 * threadIdx.x;
  if (e0 >= (uint64_t)T * H) return;
  const uint32_t t = (uint32_t)(e0 / H), i = (uint32_t)(e % H);
  if (threadIdx.x < kHcStreams4)
    ws[threadIdx.x] = __fmul_rn(2.0f, sigmoid_libm(__fmul_rn(inj[(uint64_t)t * kHcStreams4 + threadIdx.x], 0.25f), tab));
  const float2 yv = *(const float2 *)(y + e);
  float2 rv[kHcStreams4];
#pragma unroll
  for (uint32_t s = 0; s < kHcStreams4; s++) rv[s] = *(const float2 *)(R + ((uint64_t)t * kHcStreams4 + s) * H + i);
  __syncthreads();
#pragma unroll
  for (uint32_t s = 0; s < kHcStreams4; s++) {
    const float w = ws[s];
    *(float2 *)(R + ((uint64_t)t * kHcStreams4 + s) * H + i) =
        make_float2(__fadd_rn(rv[s].x, __fmul_rn(w, yv.x)), __fadd_rn(rv[s].y, __fmul_rn(w, yv.y)));
  }
}

}  // namespace

hipError_t prefill_hc_pre(const HcShape &S, const HcLayer &L, const HcBufs &b, const float *R, bool force_open,
                          hipStream_t st) {
  const uint32_t H = S.H, lr = S.lr, T = S.T, D = kHcStreams4 * H, Md = lr + kHcStreams4;
  pf_hc_norm<<<T, kHcWG, 0, st>>>(R, L.gamma, H, b.sc, b.nb, b.nn, b.nlsb, b.cnt);
  // The down GEMM: K = 4H in kHcDownSplit parts. Roundings on a sum's path: here at most 4 per matrix-core step over a
  // kGroupK chain, one per group total, one per split; in the fixed order 8 (chain) + 1 + 3 (tree) + K / 2048 (the
  // slot's chunks) + 16 (the slots); doubled, and 2^-53 each.
  const uint32_t ksplit = (D / kHcDownSplit + kGroupK - 1) / kGroupK * kGroupK;
  const double nd = 2.0 * (4.0 * (kGroupK / 4) + D / kGroupK + kHcDownSplit + 28.0 + D / 2048.0);
  const dim3 gd(((Md + 63) / 64) * ((T + 63) / 64), kHcDownSplit);
  pf_hc_gemm<false><<<gd, kHcWG, 0, st>>>(L.w_down, lr, L.w_inj, Md, D, b.nb, T, ksplit, b.part, nullptr, nullptr,
                                          nullptr, nullptr, nullptr, 0.0, nullptr, nullptr);
  pf_hc_down_fin<<<T, kHcWG, 0, st>>>(b.part, T, Md, kHcDownSplit, L.row_norm, b.nn, L.row_lsb, b.nlsb,
                                      nd * 0x1p-53, force_open, b.raw, b.open, b.cnt);
  pf_hc_down_fix<<<256, kHcWG, 0, st>>>(L.w_down, L.w_inj, lr, D, b.nb, b.open, b.cnt, b.raw);
  pf_hc_down_epi<<<T, kHcWG, 0, st>>>(b.raw, lr, b.lb, b.inj, b.ln, b.llsb);
  // The up GEMM: 4H rows of W_up against bf16(l), K = lr; the fixed order is a k chain of lr terms.
  const double nu = 2.0 * (4.0 * (kGroupK / 4) + lr / (double)kGroupK + 1.0 + lr);
  const dim3 gu(((D + 63) / 64) * ((T + 63) / 64), 1);
  pf_hc_gemm<true><<<gu, kHcWG, 0, st>>>(L.w_up, D, nullptr, D, lr, b.lb, T, lr, nullptr, b.a, L.row_norm + Md, b.ln,
                                         L.row_lsb + Md, b.llsb, nu * 0x1p-53, b.open_up, b.cnt + 1);
  pf_hc_up_fix<<<256, kHcWG, 0, st>>>(L.w_up, lr, D, b.lb, b.open_up, b.cnt + 1, b.a);
  const uint64_t nx = (uint64_t)T * H;
  pf_hc_mix<<<(uint32_t)((nx + 2 * kHcWG - 1) / (2 * kHcWG)), kHcWG, 0, st>>>(R, L.gamma, b.sc, b.a, T, H, b.x);
  return hipGetLastError();
}

hipError_t prefill_hc_post(const HcShape &S, const HcBufs &b, float *R, const float *y, hipStream_t st) {
  const uint64_t nx = (uint64_t)S.T * S.H;
  pf_hc_post<<<(uint32_t)((nx + 2 * kHcWG - 1) / (2 * kHcWG)), kHcWG, 0, st>>>(R, y, b.inj, S.T, S.H);
  return hipGetLastError();
}

}  // namespace c0ven
