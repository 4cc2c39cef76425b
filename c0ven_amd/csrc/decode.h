// What the decode kernels take: one struct by value (the kernel-argument segment), filled by the host per call.
#pragma once

#include <stdint.h>

#include "../../include/c0ven_moe_tile.h"

namespace c0ven {

constexpr uint32_t kMaxExperts = 512;     // routed experts a layer may have
constexpr uint32_t kMaxUsed = 16;         // k
constexpr uint32_t kMaxDecodeTokens = 16; // tokens the decode path takes per call
constexpr uint32_t kMaxUnits = 32;        // 256-value units per row: H and F up to 8192

// Groups one decode call can make: every assignment its own group, and the shared expert's.
constexpr uint32_t max_groups(uint32_t T, uint32_t K) { return T * K + (T + MOE_GROUP_MAX - 1) / MOE_GROUP_MAX; }

struct DecodeParams {
  uint32_t H, F, E, K, T;
  uint32_t gate_type, down_type, sh_gate_type, sh_down_type, has_shared;
  uint32_t xact_r, xact_s;  // the activation types x is quantised to for the routed and the shared gate
  float swiglu_limit;
  uint32_t route;          // 1: route x; 0: the host gave ids, w and the groups (pre-routed jobs); x is only quantised
  const uint32_t *tok_need;  // pre-routed: outputs token t sums (its jobs); null: K + has_shared
  // The layer.
  const uint16_t *router;  // (E + 1) x H bf16, the last row the shared gate
  const float *bias;       // E, or null
  const uint8_t *experts;  // routed expert e at experts + e * ex_bytes: gate, then up at ex_up_off, down at ex_down_off
  uint64_t ex_bytes, ex_up_off, ex_down_off;
  const uint8_t *shared;   // the shared expert, laid out the same with its own types
  uint64_t sh_up_off, sh_down_off;
  // Input and output: T x H fp32, rows contiguous.
  const float *x;
  float *y;
  // Scratch (sized for kMaxDecodeTokens at open).
  uint8_t *act_r, *act_s;  // T x (H / 256) activation units; act_s == act_r when the two types agree
  float *logits;           // T x (E + 1)
  int32_t *ids;            // T x K
  float *w;                // T x K
  float *gs;               // T
  MoeGroup *groups;
  uint32_t *ngroups;
  float *h;                // (T K + T) x F: SwiGLU of each assignment, fp32
  float *y_asg;            // (T K + T) x H: each assignment's expert output
  uint32_t *cnt_route;     // 1
  uint32_t *cnt_tok;       // T x (H / kDownRows): outputs in per (token, down row block)
};

// Work-group shapes. moe_gate_up: four waves, a lane one (row, unit) pair of gate or up, so a wave holds
// 32 / U rows of both; moe_down: two waves, a lane one (row, unit) pair, 64 / U_down rows a wave.
constexpr uint32_t kGateUpWG = 256, kDownWG = 128;
constexpr uint32_t gate_up_rows(uint32_t Ug) { return (kGateUpWG / 64) * (32 / Ug); }
constexpr uint32_t down_rows(uint32_t Ud) { return (kDownWG / 64) * (64 / Ud); }

__global__ void moe_route(DecodeParams p);
__global__ void moe_gate_up(DecodeParams p);
__global__ void moe_down(DecodeParams p);

}  // namespace c0ven
