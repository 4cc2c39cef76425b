// The prefill path of the MoE block (more tokens than the decode kernel takes): its shapes, buffers and launcher.
//
// Replaces the reference's prefill kernel list for the block (prompt.cpp:609-655): p_router (prompt.cl:653-679),
// p_moe_count / p_moe_scan / p_moe_fill / p_moe_scatter (prompt.cl:682-755), moe_gate_up_t (qgemm.cl:88-161),
// moe_down_t (qgemm.cl:227-239) and p_moe_combine (prompt.cl:769-787). Kernels, in stream order:
//   pf_quant_rows  x -> the experts' activation units (q8_K or q8_0, the CPU rules)
//   pf_router      logits = bf16(W) bf16(x) summed in fp64 in k order (each product exact), rounded once, + bias
//   pf_topk        one wave a token: softmax, top k, weights, shared gate; each choice's bit in its window's mask
//                  (by default instead: pf_xprep, pf_router_bf16 on the bf16 matrix cores within a stated bound, and
//                  pf_topk_cert, which sums exactly the experts the bound leaves open: ids the same)
//   pf_place       counting sort of the T k assignments by expert (stable: token order within an expert) into
//                  MoeTile[] of at most MOE_TILE rows, perm (position -> assignment) and inv (assignment -> position)
//                  (pre-routed ids: pf_masks builds the masks first)
//   gate/up        per tile: gate and up on int8 MFMA, exact int32 block sums, the blocks' integer scales and the
//                  unit's fp32 term in the oracle's order, SwiGLU. Q4_K: pf_gate_up_q4k, IQ3_S: pf_gate_up_iq3s (64
//                  rows of each a work-group); the other types: pf_gemm16 (32 rows of each); activations loaded
//                  straight to LDS
//   pf_quant_rows  h -> the down's activation units
//   down           per tile: the same kernels (64 or 128 rows a work-group)
//   pf_combine     y_t = sum_k w_k y_(t,k) in rank order + gs_t s_t
// The shared expert runs through the same GEMMs over the tokens in order.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/c0ven_moe_tile.h"

namespace c0ven {

struct PfShape {
  uint32_t H, F, E, K, T;
  uint32_t gate_type, down_type, sh_gate_type, sh_down_type, has_shared;
  float swiglu_limit;
  uint32_t sh_up_type;  // the shared expert's up; when it is not sh_gate_type, gate and up run as two GEMMs
  uint32_t exact_router;  // 1: the router's fp64 k-order sums for every logit (pf_router); 0: bf16 matrix cores and
                          // certified top-k (pf_router_bf16, pf_topk_cert)
};

struct PfLayer {
  const uint16_t *router;  // (E + 1) x H bf16
  const uint16_t *router_t;  // its E routed rows again in 16 x 32 tiles (the matrix-core router's operand)
  const float *bias;       // E or null
  const uint8_t *experts;  // expert e at experts + e * ex_bytes (gate, up at ex_up_off, down at ex_down_off)
  uint64_t ex_bytes, ex_up_off, ex_down_off;
  const uint8_t *shared;
  uint64_t sh_up_off, sh_down_off;
  const uint8_t *codebooks;  // the caller's codebooks (QGRID layout) for IQ3_XXS and IQ2_S
  const int *rlsb;           // per routed row: the least lsb of its bf16 values (the exact-sum condition)
  float rmax;                // the largest ||W_e||_2 over the routed rows (bf16 values), rounded up
  float bias_max;            // the largest |bias_e| (0 without a bias)
};

// Scratch for up to Tmax tokens (allocated at open).
struct PfBufs {
  uint8_t *act_r, *act_s;  // Tmax x (H / 256) activation units (act_s == act_r when the types agree)
  float *logits;           // Tmax x (E + 1)
  uint16_t *xb;            // Tmax x H: bf16(x), for the matrix-core router
  uint16_t *xt;            // the same in 16 x 32 tiles (rows rounded up to 16)
  float *xn;               // Tmax: ||bf16(x_t)||_2, rounded up
  int *xlsb;               // Tmax: the least lsb of bf16(x_t)'s values
  uint32_t *cnt_exact;     // tokens whose top-k needed exact sums (accumulates until read)
  int32_t *ids;            // Tmax x K
  float *w, *gs;           // Tmax x K, Tmax
  uint32_t *perm, *inv;    // Tmax K
  MoeTile *tiles;          // Tmax K / MOE_TILE + E
  uint32_t *ntiles;        // 1
  unsigned long long *masks;  // windows x E: the tokens of each 64-token window that chose each expert
  float *h, *h_sh;         // Tmax K x F (expert order), Tmax x F
  float *h_sh_up;          // Tmax x F: the shared up's rows when its type differs from the gate's (h_sh holds gate's)
  uint8_t *hact, *hact_sh; // the same rows quantised, (F / 256) units each
  float *y_asg, *y_sh;     // Tmax K x H (expert order), Tmax x H
  // With a shared expert, the x quantiser and the shared expert's launches run on `side` (default priority), forked at
  // the start and joined before the combine, so they overlap the router instead of preceding or following the routed
  // ones; the routed launches wait for xq (the quantiser done) after the top-k.
  hipStream_t side;
  hipEvent_t fork, join, xq;
};

// Called around every kernel launch (timing); may be null.
struct PfHook {
  void (*fn)(void *ctx, const char *kernel, int after, hipStream_t s);
  void *ctx;
};

constexpr uint32_t pf_max_tiles(uint32_t T, uint32_t K, uint32_t E) { return (T * K + MOE_TILE - 1) / MOE_TILE + E; }
// 64-token windows of the dispatch's masks.
constexpr uint32_t pf_windows(uint32_t T) { return (T + 63) / 64; }

// Enqueues the block for s.T tokens of x (T x H fp32, rows contiguous, device) into y (the same shape); returns the
// launches' error state.
hipError_t prefill_forward(const PfShape &s, const PfLayer &L, const PfBufs &b, const float *x, float *y, hipStream_t st,
                     const PfHook &hook);
// Pre-routed (CpuExperts::compute_many's jobs): b.ids and b.w already hold s.T x s.K ranks (ids < 0 where a token has
// fewer jobs; s.K at most the scratch's width); no router, no shared expert. y[t] = the token's jobs in rank order.
hipError_t prefill_jobs(const PfShape &s, const PfLayer &L, const PfBufs &b, const float *x, float *y, hipStream_t st,
                        const PfHook &hook);

}  // namespace c0ven
