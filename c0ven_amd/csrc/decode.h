// What the decode kernel takes: one struct by value (the kernel-argument segment), filled by the host per call.
#pragma once

#include <stdint.h>

#include "../../include/c0ven_moe_tile.h"
#include "../../include/c0ven_quant.h"
#include "layout.h"

namespace c0ven {

constexpr uint32_t kMaxExperts = 512;      // routed experts a layer may have
constexpr uint32_t kMaxUsed = 16;          // k
constexpr uint32_t kMaxDecodeTokens = 16;  // tokens the decode path takes per call
constexpr uint32_t kMaxUnits = 32;         // 256-value units per row: H and F up to 8192

// Groups one decode call can make: every assignment its own group, and the shared expert's.
constexpr uint32_t max_groups(uint32_t T, uint32_t K) { return T * K + (T + MOE_GROUP_MAX - 1) / MOE_GROUP_MAX; }

// The work-group (four waves) and the work items of moe_decode, in the order every work-group walks them:
//   lead items       when routing: items t < T quantise x[t] (to the experts' activation types), the next ones
//                    kRouteRows router rows each (a 512-value chunk a wave); without routing, items t < T quantise
//                    x[t];
//   top-k items      one a token (when routing): the shared gate's row, then softmax, top-k and weights;
//   shared items     (when routing with a shared expert) the shared expert's gate/up then down items, for each chunk
//                    of MOE_GROUP_MAX tokens: they need no routing, so they run beside the router;
//   gate/up items    gate_up_rows(U) rows of gate and of up of one routed group, all units (wave w: matrix w % 2,
//                    rows (w / 2) 64 / U .., lane = r * U + u);
//   down items       down_rows(U_down) rows of down of one routed group (lane = r * U_down + u);
//   combine items    one a (token, down row block): the token's outputs summed in rank order (after all down items).
constexpr uint32_t kWG = 256;
#ifndef C0VEN_ROUTE_ROWS
#define C0VEN_ROUTE_ROWS 1
#endif
constexpr uint32_t kRouteRows = C0VEN_ROUTE_ROWS;  // router rows a lead item (x read once for all of them)
constexpr uint32_t lead_items(uint32_t T, uint32_t E, uint32_t route) {
  return route ? T + (E + kRouteRows - 1) / kRouteRows : T;
}
constexpr uint32_t kMaxLeadItems = kMaxDecodeTokens + kMaxExperts;
// LDS a lead item's dot products take from the dynamic allocation: 16 partials and the total of each (row, token).
constexpr uint32_t kRouterLds = kRouteRows * kMaxDecodeTokens * 17 * 8;
// Chunks of the shared expert's tokens (one group's worth each) when it runs beside the router.
constexpr uint32_t shared_chunks(uint32_t T, uint32_t route, uint32_t has_shared) {
  return route && has_shared ? (T + MOE_GROUP_MAX - 1) / MOE_GROUP_MAX : 0;
}
// Groups a launch may have: routed (every assignment its own, at worst), or a pre-routed call's jobs.
constexpr uint32_t kMaxGroups = max_groups(kMaxDecodeTokens, kMaxUsed + 1);
// LDS the grouping step takes from the dynamic allocation: T K ids, a token mask and two group numbers per expert,
// and a count of heads per wave and group size.
constexpr uint32_t kGroupingLds =
    kMaxDecodeTokens * kMaxUsed * 4 + kMaxExperts * 4 + kMaxExperts * 2 * 4 + (kWG / 64) * MOE_GROUP_MAX * 4;
constexpr uint32_t kDynLists = 8;     // lists the routed items are dealt from (one counter each)
constexpr uint32_t kDynStride = 64;   // words between two list counters
// LDS after a group's activation units for the matrix-core gate/up item's exchanges (unit terms, then sums).
constexpr uint32_t kMfmaXchBytes = (2 * 4 * 4 * 64 + 2 * 16 * 16) * 4;
constexpr uint32_t gate_up_rows(uint32_t Ug) { return (kWG / 64) * (32 / Ug); }
// Bytes between two tokens' activation units in LDS (a token's U units are kActLds apart): padded to an odd multiple
// of 8 words modulo 32 banks, so that the matrix-core B operand's 16 tokens x 4 eight-byte pieces read at the
// 4-way minimum (U = 8 unpadded puts every token on the same bank).
constexpr uint32_t act_tok_stride(uint32_t U) {
  return (U * (kActLds / 4) + (24 - (U * (kActLds / 4)) % 16) % 16) * 4;
}
static_assert(act_tok_stride(8) % 128 == 32 && act_tok_stride(2) == 2 * kActLds, "activation token stride");
// LDS after the activation units in which a dot4 gate/up item's up waves hand their row sums to the gate waves.
constexpr uint32_t gate_up_xch_bytes(uint32_t Ug) { return gate_up_rows(Ug) * MOE_GROUP_MAX * 4; }
constexpr uint32_t down_rows(uint32_t Ud) { return (kWG / 64) * (64 / Ud); }

// Flags (64-bit, set to the launch's epoch): [i < kMaxLeadItems] lead item i is done (its quantised x is in, for
// the shared expert's items), [kFlagRouted] a pre-routed call's x is quantised. Data handed from one work item to the
// next inside a launch (logits, ids, weights, the shared gate, h) travels as tagged records instead: 64-bit words
// whose high half is the launch's tag, so the reader polls the data itself and needs no flag.
// With the hyper-connection mix (hc_R not null): [kFlagHcNorm + 4 t + s] token t's stream s is normed, [kFlagHcDown] the
// low-rank gate and the inject logits are in, [kFlagHcX] the mixed input x is in.
constexpr uint32_t kFlagLead = 0, kFlagRouted = kMaxLeadItems, kFlagHcNorm = kMaxLeadItems + 1,
                   kFlagHcDown = kFlagHcNorm + 4 * kMaxDecodeTokens, kFlagHcX = kFlagHcDown + 1,
                   kFlagCount = kFlagHcX + 1;

// The hyper-connection mix before the block and the combine after it (docs/spec/MODEL_LAYER.md 1.1, 1.2): 4 streams
// of H values a token, a low rank of at most kHcMaxLr. Its items come first in a launch:
//   norm items      one a token's stream: its RMS norm (x gamma);
//   down items      one a row of W_down (lr rows) and of W_inject (4 rows), for all tokens: silu(W_down n / 4), and
//                   the inject logits W_inject n;
//   up items        kHcUpValues values of x, for all tokens: the 4 kHcUpValues rows of W_up they take, then the mix.
// The lead items wait for x; the combine items add the block's output into the streams.
constexpr uint32_t kHcStreams = 4, kHcMaxLr = 512, kHcUpValues = 16;
constexpr uint32_t hc_items(uint32_t T, uint32_t H, uint32_t lr) {
  return lr ? kHcStreams * T + lr + kHcStreams + H / kHcUpValues : 0;
}

struct DecodeParams {
  uint32_t H, F, E, K, T;
  uint32_t gate_type, down_type, sh_gate_type, sh_down_type, has_shared;
  uint32_t sh_up_type;       // the shared expert's up (its gate's activation type; a grid type only if equal to gate's)
  uint32_t xact_r, xact_s;  // the activation types x is quantised to for the routed and the shared gate
  float swiglu_limit;
  uint32_t route;            // 1: route x; 0: the host gave ids, w and the groups (pre-routed jobs)
  const uint32_t *tok_need;  // pre-routed: outputs token t sums (its jobs); null: K + has_shared
  uint64_t epoch;            // this launch's number: a flag is set when it holds it
  uint32_t tag;              // its low 32 bits: a tagged record (value in the low word) is valid when it holds it
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
  // Scratch (sized for max_tokens at open). Everything written here during a launch and read by another work-group
  // goes through device-coherent stores and loads.
  uint8_t *act_r, *act_s;  // T x (H / 256) activation units; act_s == act_r when the two types agree
  uint64_t *logits;        // T x (E + 1) tagged records (the fp32 bits)
  int32_t *ids;            // T x K: the routed ids as the caller reads them, or a pre-routed call's
  float *w;                // T x K: the same for the weights
  uint64_t *ids_t, *w_t;   // T x K tagged records of the routed ids and weights
  uint64_t *gs;            // T tagged records: the shared expert's gate
  MoeGroup *groups;
  uint32_t *ngroups;
  uint64_t *h;             // (T K + T) x F tagged records: SwiGLU of each assignment, fp32
  uint64_t *y_asg;         // (T K + T) x H tagged records: each assignment's expert output
  uint64_t *flags;         // kFlagH + G
  uint32_t *cnt_route;     // 1: lead items in (pre-routed calls)
  uint32_t *cnt_topk;      // 1: tokens routed
  uint32_t *cnt_dyn;       // 2 x kDynLists counters, kDynStride apart: the routed items' lists (alternate launches)
  uint32_t *err;           // set when a wait gave up (never, unless a work-group could not run)
  uint64_t *trace;         // null, or (start, ready, computed, end) s_memrealtime stamps per work item
  uint32_t trace_cap;
  const uint8_t *codebooks;  // the caller's codebook buffer (QGRID layout) on the device, or null
  // The hyper-connection mix and combine (hc_R null: off; x is then the caller's).
  float *hc_R;               // T x 4 x H: the residual streams, read by the mix, added to by the combine
  const float *hc_gamma;     // 4 H: the streams' norm weights
  const uint16_t *hc_down;   // lr x 4 H bf16
  const uint16_t *hc_inj;    // 4 x 4 H bf16
  const uint16_t *hc_up;     // 4 H x lr bf16 (row s H + i), then its rows' 2-norms (4 H fp64, rounded up) and least
                             // lsb exponents (4 H int)
  uint32_t hc_lr;
  float *hc_n;               // the normed streams as bf16 (T x 4 H), then the norms' scales (T x 4 fp32)
  float *hc_l;               // T x (lr + 4): the gate silu(W_down n / 4), then the inject logits
  float *hc_x;               // T x H: the mixed input (x points here)
  uint32_t *cnt_hc;          // 2 counters, kDynStride words apart: down items in, up items in
  // Experts not on the device (core/models/qwen4exp/layout.h:64-71, layer.cl:838-884): a routed expert e with
  // resident[e] == 0 is a miss. Its assignment joins no group; the top-k item publishes the token's misses in its
  // record in host memory (miss_jobs, behind a system-scope release of the step number), and the token's combine items
  // wait (bounded) for the host's answer (ans_seq == the step) and add ans_y's row after the shared expert's term.
  const uint8_t *resident;   // E flags, or null: every expert is on the device
  uint8_t *miss_jobs;        // a moe_miss_job record a token, miss_stride bytes apart (host memory), or null
  uint32_t miss_stride;
  const float *ans_y;        // T x H (host memory): the host's sum over each token's misses
  const uint32_t *ans_seq;   // (host memory): the step whose answer ans_y holds
};

// The weight types a launch may meet, as a set (bits below): moe_decode is compiled once per set, so a context whose
// matrices share one type carries no other type's code (and no register pressure from it). kTypeQ8_0 stands for the
// 32-value block types that meet q8_0 activations (Q8_0, IQ4_NL, Q2_0), which differ only in how a unit decodes,
// kTypeQ4_K for the q8_K types without a codebook (Q4_K, Q5_K, Q6_K, IQ4_XS) and kTypeIQ2 for the codebook types
// (IQ3_XXS, IQ2_S).
constexpr uint32_t kTypeQ8_0 = 1, kTypeQ4_K = 2, kTypeIQ3_S = 4, kTypeIQ2 = 8;
constexpr uint32_t type_bit(uint32_t qt) {
  return (qt == QT_Q8_0 || qt == QT_IQ4_NL || qt == QT_Q2_0) ? kTypeQ8_0
         : kq_family(qt)                                     ? kTypeQ4_K
         : qt == QT_IQ3_S                                    ? kTypeIQ3_S
                                                             : kTypeIQ2;
}
// Words of LDS a grid type's codebook takes (IQ2_S: 1024 entries of two words).
constexpr uint32_t kGridWords = 2048;

// The activation type (q8_0 for Q8_0 weights, q8_K for the others), fixed at compile time where the set allows.
template <uint32_t kTypes>
__device__ __forceinline__ uint32_t act_type(uint32_t runtime) {
  if constexpr (kTypes == kTypeQ8_0) return QT_Q8_0;
  if constexpr ((kTypes & kTypeQ8_0) == 0) return QT_Q8_K;
  return runtime;
}

template <uint32_t kTypes, bool kHc>
__global__ void moe_decode(DecodeParams p);

// The instantiation for a type set (1 .. 15), with the hyper-connection items or not, as a kernel handle for
// hipLaunchKernel.
const void *decode_kernel(uint32_t types, bool hc);

}  // namespace c0ven
