// The hyper-connection mix and combine around the prefill block (more tokens than the decode kernel takes): the
// kernels of moe_prefill_hc.hip and what they take.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace c0ven {

struct HcShape {
  uint32_t H, lr, T;  // n_embd, the low rank (a multiple of 8), tokens
};

// One layer's module on the device: gamma (4 H fp32), W_down (lr x 4H bf16), W_inject (4 x 4H), W_up (4H x lr), the
// 2-norms of their rows (W_down's and W_inject's lr + 4, then W_up's 4H; fp64, rounded up) and the least lsb exponent
// of each row's nonzero values (same order; a bf16 value with exponent field e > 0 has lsb 2^(e - 134)).
struct HcLayer {
  const float *gamma;
  const uint16_t *w_down, *w_inj, *w_up;
  const double *row_norm;
  const int *row_lsb;
};

// Scratch for T tokens: the norm's scales (T x 4) and the normed streams' bf16 bits (T x 4 x H), their bf16 2-norms,
// the down GEMM's fp64 partials (kHcDownSplit x T x (lr + 4)) and rounded sums (T x (lr + 4)), the list of sums whose
// rounding the bound left open (pairs t, row; room for all) and the up GEMM's, their counts, bf16(l) (T x lr) and its
// norms, the inject logits (T x 4), the up GEMM's sums a (T x 4H), and x (T x H).
struct HcBufs {
  float *sc, *raw, *inj, *a, *x;
  uint16_t *nb, *lb;  // bf16(n), bf16(l): the GEMMs' operands
  double *nn, *ln, *part;
  int *nlsb, *llsb;  // the least lsb exponent of each token's bf16(n), bf16(l)
  uint32_t *open, *open_up, *cnt;  // cnt[0]: open's entries (down), cnt[1]: open_up's (up; room for T x 4H)
};

constexpr uint32_t kHcDownSplit = 8;  // K parts of the down GEMM: its grid then fills the device (4: 494, 16: 459, 8: 453 us)

// R (T x 4 x H, device) to the block's input x (bufs.x) and the inject logits; force_open (tests) sends every down
// sum through the exact-order recomputation.
hipError_t prefill_hc_pre(const HcShape &S, const HcLayer &L, const HcBufs &b, const float *R, bool force_open,
                          hipStream_t st);
// R_s += 2 sigma(inject_s / 4) y.
hipError_t prefill_hc_post(const HcShape &S, const HcBufs &b, float *R, const float *y, hipStream_t st);

}  // namespace c0ven
