// The decode-shape MoE block (a few tokens: decode and speculative verify) as one persistent kernel.
//
// Replaces the reference's decode kernel list for the block (model.cpp:1348-1414): the router's bf16 GEMV
// (mv_xmx_bf16), router_group (layer.cl:984-1023), moe_gate_up_g (moe.cl:230-302), moe_down_g (moe.cl:416-471) and
// moe_combine (layer.cl:869-884). Every work-group walks the work items b, b + grid, b + 2 grid, ... in one order
// (decode.h): lead items (x quantised; router rows), top-k items, the shared expert's items; then it takes the routed
// gate/up, down and combine items from the list of its index modulo 8 (a counter a list). An item that needs earlier
// work waits for it (flags set to this launch's epoch, or tagged records whose tag is this launch's):
//   - an x item sets its token's flag; a top-k item polls the logits the lead items store;
//   - every work-group builds the routed groups from the ids the top-k items store;
//   - a down item polls its group's h, a combine item the outputs of its token's assignments.
// Every item's dependencies have smaller indices. Progress: lead items wait for nothing; the dispatcher deals a grid's
// work-groups to the eight XCDs in turn (work-group b to XCD b mod 8) and each XCD starts its share in index order,
// so a work-group never waits behind a later one of its own XCD, and list x is served by XCD x's work-groups, which
// take its items in order. So the smallest unfinished item always progresses once its XCD admits any work-group of
// this kernel, whatever else the device runs and however large the grid (a multiple of 8; moe_set_grid). Waits are
// bounded anyway: past kSpinLimit polls (seconds) a wait gives up and sets *err.
#include <hip/hip_runtime.h>

#include <type_traits>

#include "../../include/c0ven_moe.h"
#include "act_quant.h"
#include "decode.h"
#include "route.h"
#include "device_math.h"
#include "iq3s_grid.h"
#include "layout.h"
#include "mfma_q4k.h"
#include "units.h"

namespace c0ven {

__device__ __constant__ static const uint32_t kIq3sGridDev[512] = {C0VEN_IQ3S_GRID_VALUES};

namespace {

constexpr uint32_t kSpinLimit = 1u << 22;
#ifndef C0VEN_POLL_SLEEP
#define C0VEN_POLL_SLEEP 1
#endif

// The thread index, read afresh where it is used: the empty asm hides that it is the same value everywhere, so the
// compiler recomputes addresses derived from it at their use instead of hoisting them out of the item loop, where the
// kernel's register pressure would spill them to scratch (each reload a memory round trip in a hand-off).
__device__ __forceinline__ uint32_t tid() {
  uint32_t t = threadIdx.x;
  asm volatile("" : "+v"(t));
  return t;
}
__device__ __forceinline__ uint32_t lane_id() { return tid() & 63u; }
__device__ __forceinline__ uint32_t wave_id() { return tid() >> 6; }

// This work-group's coherent stores are complete (every wave waits for its own, then the barrier).
__device__ __forceinline__ void stores_done() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
}

// Counts the work-group in on *cnt once its stores are complete; true in every thread of the one that completes
// `total` (which sets the counter back to zero for the next launch).
__device__ __forceinline__ bool arrive_last(uint32_t *cnt, uint32_t total, uint32_t *flag) {
  stores_done();
  if (tid() == 0) {
    const uint32_t old = __hip_atomic_fetch_add(cnt, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    *flag = old == total - 1;
    if (old == total - 1) __hip_atomic_store(cnt, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  __syncthreads();
  return *flag != 0;
}

// Sets flag i to this launch's epoch once the work-group's stores are complete.
__device__ __forceinline__ void set_flag(const DecodeParams &p, uint32_t i) {
  stores_done();
  if (tid() == 0) st_co(p.flags + i, p.epoch);
}

// Waits until flag i holds this launch's epoch (thread 0 polls, the work-group follows).
__device__ __forceinline__ void wait_flag(const DecodeParams &p, uint32_t i) {
  if (tid() == 0) {
    uint32_t n = 0;
    while (ld_co(p.flags + i) != p.epoch) {
      __builtin_amdgcn_s_sleep(C0VEN_POLL_SLEEP);
      if (++n == kSpinLimit) {
        st_co(p.err, 1u);
        break;
      }
    }
  }
  __syncthreads();
}

// Waits until flags base .. base + count - 1 (count <= 64) all hold this launch's epoch (wave 0 polls,
// a flag a lane, all loads of a round in flight together; the work-group follows).
__device__ __forceinline__ void wait_flags(const DecodeParams &p, uint32_t base, uint32_t count) {
  if (wave_id() == 0) {
    uint32_t n = 0;
    for (;;) {
      const uint32_t f = lane_id();
      const bool ok = f >= count || ld_co(p.flags + base + f) == p.epoch;
      if (__all(ok)) break;
      __builtin_amdgcn_s_sleep(1);
      if (++n == kSpinLimit) {
        if (lane_id() == 0) st_co(p.err, 1u);
        break;
      }
    }
  }
  __syncthreads();
}

// The value of a tagged record once it holds this launch's tag (the calling thread polls; past kSpinLimit polls it
// gives up, sets *err and returns what it has).
__device__ __forceinline__ uint32_t poll_tag(const DecodeParams &p, const uint64_t *q) {
  uint64_t v = ld_tag(q);
  uint32_t n = 0;
  while (tag_of(v) != p.tag) {
    __builtin_amdgcn_s_sleep(C0VEN_POLL_SLEEP);
    if (++n == kSpinLimit) {
      st_co(p.err, 1u);
      break;
    }
    v = ld_tag(q);
  }
  return (uint32_t)v;
}

// Waits (thread 0 polls, the work-group follows) until one tagged record holds this launch's tag: the cheap first
// wait before a work-group reads a whole set of records written at about the same time (each read still checks its own
// tag), so that hundreds of work-groups do not poll the whole set.
__device__ __forceinline__ void wait_tag(const DecodeParams &p, const uint64_t *q) {
  if (tid() == 0) (void)poll_tag(p, q);
  __syncthreads();
}

// Token t's logits as order keys, lane l holding experts l + 64 i: the wave polls the tagged records (the router rows'
// fp32 sums) until every one holds this launch's tag (the lead items' stores are the hand-off; no flag), then adds
// the bias.
__device__ __forceinline__ void load_logits(const DecodeParams &p, uint32_t t, uint32_t key[kRoutePer], uint32_t id[kRoutePer]) {
  const uint32_t lane = lane_id(), E = p.E;
  const uint64_t *lg = p.logits + (uint64_t)t * (E + 1);
  float bias[kRoutePer];  // read before the polling, added to the polled sums (the router rows' own fp32 add)
#pragma unroll
  for (int i = 0; i < kRoutePer; i++) bias[i] = p.bias ? p.bias[min(lane + 64 * i, E - 1)] : 0.0f;
  uint64_t v[kRoutePer];
  for (uint32_t n = 0;; n++) {
    bool ok = true;
#pragma unroll
    for (int i = 0; i < kRoutePer; i++) {
      const uint32_t e = lane + 64 * i;
      v[i] = ld_tag(lg + min(e, E - 1));
    }
#pragma unroll
    for (int i = 0; i < kRoutePer; i++) ok &= tag_of(v[i]) == p.tag;
    if (__all(ok)) break;
    __builtin_amdgcn_s_sleep(C0VEN_POLL_SLEEP);
    if (n == kSpinLimit) {
      if (lane == 0) st_co(p.err, 1u);
      break;
    }
  }
#pragma unroll
  for (int i = 0; i < kRoutePer; i++) {
    const uint32_t e = lane + 64 * i;
    const float l = __uint_as_float((uint32_t)v[i]);
    key[i] = e < E ? float_key(p.bias ? __fadd_rn(l, bias[i]) : l) : 0u;
    id[i] = e;
  }
}

// Top-k and weights for token t (route.h:39-99 and layer.cl:765-804 restated). Every wave loads the token's logits
// (lane l holds experts l + 64 i). Wave 0 selects the top k (route_select_lds: a threshold, then the candidates
// ranked in LDS). Waves 1..3 meanwhile take the softmax's max and a third of its sum each (in double); the sum is
// their three parts in order. Then wave 0 turns the k winners into weights and stores ids and w.
__device__ __forceinline__ void route_token(const DecodeParams &p, uint32_t t, const uint64_t *tab, double *dpart,
                                            uint2 *cand) {
  const uint32_t lane = lane_id(), wv = wave_id(), E = p.E, K = p.K;
  uint32_t key[kRoutePer], id[kRoutePer];
  load_logits(p, t, key, id);
  const float mx = route_max(key);
  uint32_t my_id = 0, my_key = 0;
  if (wv == 0) {
    route_select_lds(key, id, K, lane, cand, &my_id, &my_key);
    // The ids first: the groups wait for them; the weights are read only by the combine items.
    if (lane < K) st_tag(p.ids_t + t * K + lane, my_id, p.tag);
  } else {
    const double part = route_sum_part(key, E, lane, wv - 1, mx, tab);
    if (lane == 0) dpart[wv - 1] = part;
  }
  __syncthreads();
  uint32_t *nm = (uint32_t *)dpart + 8;
  if (wv == 0) {
    const float inv = (float)(1.0 / __dadd_rn(__dadd_rn(dpart[0], dpart[1]), dpart[2]));
    const float w = route_weight(my_key, mx, inv, K, lane, tab);
    if (lane < K) {
      st_tag(p.w_t + t * K + lane, __float_as_uint(w), p.tag);
      p.ids[t * K + lane] = (int32_t)my_id;  // the caller's copies, read after the launch
      p.w[t * K + lane] = w;
    }
    if (p.miss_jobs) {  // the token's record: the misses in rank order (layer.cl:781-804's rt_finish)
      moe_miss_job *job = (moe_miss_job *)(p.miss_jobs + (uint64_t)t * p.miss_stride);
      const bool miss = lane < K && !p.resident[my_id];
      const uint64_t b = __ballot(miss);
      if (lane < K) job->all[lane] = (int32_t)my_id;
      if (miss) {
        const uint32_t at = __builtin_amdgcn_mbcnt_hi((uint32_t)(b >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)b, 0u));
        job->ids[at] = (int32_t)my_id;
        job->w[at] = w;
      }
      if (lane == 0) *nm = (uint32_t)__popcll(b);
    }
  }
  if (p.miss_jobs) {  // x, then nmiss and the step (rt_publish: the step last, behind a system-scope release)
    __syncthreads();
    moe_miss_job *job = (moe_miss_job *)(p.miss_jobs + (uint64_t)t * p.miss_stride);
    float *jx = (float *)(job + 1);
    if (*nm > 0)
      for (uint32_t i = tid(); i < p.H; i += kWG) jx[i] = ld_co(p.x + (uint64_t)t * p.H + i);
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "");
    __syncthreads();
    if (tid() == 0) {
      job->nmiss = *nm;
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "");
      __hip_atomic_store(&job->seq, p.tag, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_SYSTEM);
    }
  }
}

// Group g's matrix (0 gate, 1 up, 2 down) and its type.
struct GroupMat {
  const uint8_t *mat;
  uint32_t type;
  bool shared;
};

__device__ __forceinline__ GroupMat group_mat(const DecodeParams &p, int32_t slot, int which) {
  GroupMat m;
  m.shared = slot == (int32_t)p.E;
  if (m.shared) {
    m.type = which == 2 ? p.sh_down_type : which == 1 ? p.sh_up_type : p.sh_gate_type;
    m.mat = p.shared + (which == 0 ? 0 : which == 1 ? p.sh_up_off : p.sh_down_off);
  } else {
    m.type = which == 2 ? p.down_type : p.gate_type;
    m.mat = p.experts + (uint64_t)slot * p.ex_bytes + (which == 0 ? 0 : which == 1 ? p.ex_up_off : p.ex_down_off);
  }
  return m;
}

// The codebook of a grid type into LDS, unless the work-group's previous item left it there (*have: the type it holds).
__device__ __forceinline__ void load_grid(const DecodeParams &p, uint32_t type, uint32_t *grid_lds, uint32_t *have) {
  if (*have == type) return;
  if (type == QT_IQ3_S) {
    for (uint32_t i = tid(); i < 512; i += kWG) grid_lds[i] = kIq3sGridDev[i];
  } else {
    const uint32_t *src = (const uint32_t *)(p.codebooks + (type == QT_IQ2_S ? QGRID_IQ2S : QGRID_IQ3XXS));
    const uint32_t n = type == QT_IQ2_S ? 2048u : 256u;
    for (uint32_t i = tid(); i < n; i += kWG) grid_lds[i] = src[i];
  }
  __syncthreads();
  if (tid() == 0) *have = type;
  __syncthreads();
}

// The n terms of one (row, unit) pair against the activation units act + j * stride dwords, into t[j]. The unit's
// weights are loaded first; `ready` (run by the whole work-group) then makes the activations available, so the
// weights' HBM latency overlaps whatever ready waits for.
template <uint32_t kTypes, typename Ready>
__device__ __forceinline__ void pair_terms(uint32_t type, const uint8_t *tile, uint32_t idx, uint32_t nl,
                                           const uint32_t *grid_lds, const uint32_t *act, uint32_t stride,
                                           const uint32_t &n, float *t, Ready ready) {
  if constexpr ((kTypes & kTypeQ8_0) != 0) {
    if (kTypes == kTypeQ8_0 || q8_family(type)) {
      const auto run = [&](auto &w) {
#pragma unroll
        for (uint32_t j = 0; j < MOE_GROUP_MAX; j++)
          if (j < n) t[j] = w.term(Act(act + j * stride));
      };
      if (type == QT_Q2_0) {  // a branch a type, so that no two types' registers are live together
        UnitQ8Split<QT_Q2_0> w;
        w.load_raw(tile, idx, nl);
        ready();
        w.widen();
        run(w);
      } else if (type == QT_IQ4_NL) {
        UnitQ8Split<QT_IQ4_NL> w;
        w.load_raw(tile, idx, nl);
        ready();
        w.widen();
        run(w);
      } else {
        UnitQ8_0 w;
        w.load(tile, idx, nl);
        ready();
        run(w);
      }
      return;
    }
  }
  if constexpr ((kTypes & kTypeQ4_K) != 0) {
    if ((kTypes & ~kTypeQ8_0) == kTypeQ4_K || kq_family(type)) {
      const auto run = [&](auto &w) {
        w.load(tile, idx, nl);
        ready();
#pragma unroll
        for (uint32_t j = 0; j < MOE_GROUP_MAX; j++)
          if (j < n) t[j] = w.term(Act(act + j * stride));
      };
      if (type == QT_Q4_K) {  // a branch a type, so that no two types' registers are live together
        UnitQ4_K w;
        run(w);
      } else if (type == QT_Q6_K) {
        UnitQ6_K w;
        run(w);
      } else if (type == QT_IQ4_XS) {
        UnitIQ4_XS w;
        run(w);
      } else {
        UnitQ5_K w;
        run(w);
      }
      return;
    }
  }
  const auto run = [&](auto &w) {
    w.load(tile, idx, nl, grid_lds);
    ready();
#pragma unroll
    for (uint32_t j = 0; j < MOE_GROUP_MAX; j++)
      if (j < n) t[j] = w.term(Act(act + j * stride));
  };
  if constexpr ((kTypes & kTypeIQ3_S) != 0) {
    if ((kTypes & ~(kTypeQ8_0 | kTypeQ4_K)) == kTypeIQ3_S || type == QT_IQ3_S) {
      UnitIQ3_S w;
      run(w);
      return;
    }
  }
  if constexpr ((kTypes & kTypeIQ2) != 0) {
    if (type == QT_IQ3_XXS) {
      UnitIQ3_XXS w;
      run(w);
    } else {
      UnitIQ2_S w;
      run(w);
    }
  }
}

// A row's sum over its U lanes (consecutive, U a power of two, one unit each), in the oracle's order: acc = 0, then
// acc + t_u for u ascending. The partial passes one lane up at each step; every lane of the row receives the total.
__device__ __forceinline__ float row_sum(float t, uint32_t U) {
  const uint32_t lane = lane_id(), u = lane & (U - 1);
  float x = u == 0 ? __fadd_rn(0.0f, t) : t;
  for (uint32_t i = 1; i < U; i++) {
    const float prev = U <= 16 ? __uint_as_float(dpp_u32<kDppShr1>(__float_as_uint(x))) : __shfl_up(x, 1, 64);
    if (u == i) x = __fadd_rn(prev, t);
  }
  return __shfl(x, (int)((lane & ~(U - 1)) + U - 1), 64);
}


// ---------------------------------------------------------------------------------------------------------------
// Router items

// x[t] to the activation types of the routed and the shared gate: a half-wave per unit.
template <uint32_t kTypes, bool kHc>
__device__ __forceinline__ void quantise_x(const DecodeParams &p, uint32_t t) {
  const uint32_t H = p.H, l32 = tid() & 31u;
  for (uint32_t u = tid() / 32; u < H / kUnit; u += kWG / 32) {
    float4 a, b;
    const uint64_t e = (uint64_t)t * H + u * kUnit + 8 * l32;
    if constexpr (kHc) {  // x from this launch's up items
      const uint4 ua = ld_co16(p.x, (uint32_t)(4 * e)), ub = ld_co16(p.x, (uint32_t)(4 * e + 16));
      a = make_float4(__uint_as_float(ua.x), __uint_as_float(ua.y), __uint_as_float(ua.z), __uint_as_float(ua.w));
      b = make_float4(__uint_as_float(ub.x), __uint_as_float(ub.y), __uint_as_float(ub.z), __uint_as_float(ub.w));
    } else {
      a = ((const float4 *)(p.x + e))[0], b = ((const float4 *)(p.x + e))[1];
    }
    const float v[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
    quant_unit(v, l32, act_type<kTypes>(p.xact_r), p.act_r + ((uint64_t)t * (H / kUnit) + u) * kActBytes);
    if (p.act_s != p.act_r) quant_unit(v, l32, act_type<kTypes>(p.xact_s), p.act_s + ((uint64_t)t * (H / kUnit) + u) * kActBytes);
  }
}

// Eight doubles of every lane summed over the 16 lanes of its row, by halving exchanges (the partner across the row's
// mirror, then the 8-lane mirror and the quad reverse, each keeping the half of the values its lane bit picks; then
// lane ^ 1): lane l of the row receives the total of v[(l % 16) / 2].
__device__ __forceinline__ double row16_reduce8_f64(double v[8]) {
  const uint32_t l = lane_id();
  auto step = [&](auto ctrl_tag, uint32_t half, uint32_t keep_hi) {
    constexpr int kCtrl = decltype(ctrl_tag)::value;
#pragma unroll
    for (uint32_t i = 0; i < 4; i++) {
      if (i >= half) break;
      const double send = keep_hi ? v[i] : v[half + i], keep = keep_hi ? v[half + i] : v[i];
      v[i] = __dadd_rn(keep, dpp_f64<kCtrl>(send));
    }
  };
  step(std::integral_constant<int, kDppMirror>{}, 4, (l >> 3) & 1u);
  step(std::integral_constant<int, kDppHalfMirror>{}, 2, (l >> 2) & 1u);
  step(std::integral_constant<int, kDppQuadRev>{}, 1, (l >> 1) & 1u);
  return __dadd_rn(v[0], dpp_f64<kDppXor1>(v[0]));
}

// Dot products of a bf16 row W of K values (a multiple of 512) with tokens t0 .. t0 + nt - 1 (nt <= 16) of x (rows
// ldx apart; read past the caches when kCo, for x written in this launch): tot[t] = sum over the row of
// bf16(W) bf16(x), each product exact, summed in fp64. Wave w takes the 512-value chunks w, w + 4, ..., lane l values
// 8 l .. 8 l + 7 of each: a lane converts its weights once for all tokens. Eight tokens at a time (x of four in flight
// while four are used), each chunk's eight sums are reduced over the 16 lanes of a row (one value a lane pair left) and
// added to that row of lanes' partial in LDS; the sixteen partials of an output (four rows of lanes, four waves) are
// then added in a fixed order.
template <bool kCo, bool kXb = false>
__device__ __forceinline__ void bf16_dot(const uint16_t *W, const float *x, uint32_t K, uint32_t ldx, uint32_t t0,
                                         uint32_t nt, double *part, double *tot) {
  const uint32_t lane = lane_id(), wv = wave_id(), nC = K / 512;
  const uint32_t pslot = 4 * wv + lane / 16;
  // Values 8 lane .. + 7 of chunk c of token t, as two float4 (kXb: x holds bf16 bits, 16 bytes the eight).
  const auto ldx8 = [&](uint32_t t, uint32_t c, float4 &a, float4 &b) {
    const uint64_t e = (uint64_t)t * ldx + 512 * c + 8 * lane;
    if constexpr (kXb) {
      const uint4 u = ld_co16(x, (uint32_t)(2 * e));
      a = make_float4(__uint_as_float(u.x << 16), __uint_as_float(u.x & 0xffff0000u), __uint_as_float(u.y << 16),
                      __uint_as_float(u.y & 0xffff0000u));
      b = make_float4(__uint_as_float(u.z << 16), __uint_as_float(u.z & 0xffff0000u), __uint_as_float(u.w << 16),
                      __uint_as_float(u.w & 0xffff0000u));
    } else if constexpr (kCo) {
      const uint4 u = ld_co16(x, (uint32_t)(4 * e)), v = ld_co16(x, (uint32_t)(4 * e + 16));
      a = make_float4(__uint_as_float(u.x), __uint_as_float(u.y), __uint_as_float(u.z), __uint_as_float(u.w));
      b = make_float4(__uint_as_float(v.x), __uint_as_float(v.y), __uint_as_float(v.z), __uint_as_float(v.w));
    } else {
      a = ((const float4 *)(x + e))[0], b = ((const float4 *)(x + e))[1];
    }
  };
  for (uint32_t c = wv; c < nC; c += kWG / 64) {
    const uint4 wa = *(const uint4 *)(W + 512 * c + 8 * lane);
    double wd[8];
    {
      const uint32_t w0[4] = {wa.x, wa.y, wa.z, wa.w};
#pragma unroll
      for (int k = 0; k < 8; k++) wd[k] = (double)__uint_as_float((k & 1) ? w0[k / 2] & 0xffff0000u : w0[k / 2] << 16);
    }
    for (uint32_t tb = 0; tb < nt; tb += 8) {
      const uint32_t nb = min(8u, nt - tb);
      double v[8];
      float4 xq[2][4][2];
#pragma unroll
      for (uint32_t tt = 0; tt < 4; tt++) ldx8(t0 + tb + min(tt, nb - 1), c, xq[0][tt][0], xq[0][tt][1]);
#pragma unroll
      for (uint32_t tt = 0; tt < 8; tt++) {
        if (tt == 0 && nb > 4) {
#pragma unroll
          for (uint32_t u = 0; u < 4; u++) ldx8(t0 + tb + min(4 + u, nb - 1), c, xq[1][u][0], xq[1][u][1]);
        }
        double a = 0.0;
        if (tt < nb) {
          const float4 xa = xq[tt / 4][tt % 4][0], xb = xq[tt / 4][tt % 4][1];
          float xs[8];
          round_bf16_2(xa.x, xa.y, xs[0], xs[1]), round_bf16_2(xa.z, xa.w, xs[2], xs[3]);
          round_bf16_2(xb.x, xb.y, xs[4], xs[5]), round_bf16_2(xb.z, xb.w, xs[6], xs[7]);
#pragma unroll
          for (int k = 0; k < 8; k++) a = __builtin_fma(wd[k], (double)xs[k], a);
        }
        v[tt] = a;
      }
      // One tree for every token count (tokens past nb add zeros), so a token's sum does not depend on T:
      // ((P0 + P7) + (P3 + P4)) + ((P1 + P6) + (P2 + P5)), P_m = a_m + a_(15 - m) over the row's 16 lanes.
      const double s = row16_reduce8_f64(v);
      const uint32_t tt = (lane & 15u) / 2;
      if ((lane & 1u) == 0 && tt < nb) {
        double *q = part + (tb + tt) * 16 + pslot;
        *q = c == wv ? s : __dadd_rn(*q, s);
      }
    }
  }
  if (wv >= nC && (lane & 15u) == 0) {  // waves without a chunk (K < 2048) give zeros
    for (uint32_t t = 0; t < nt; t++) part[t * 16 + pslot] = 0.0;
  }
  __syncthreads();
  const uint32_t j = tid();
  if (j < nt) {
    double s = 0.0;
#pragma unroll
    for (uint32_t i = 0; i < 16; i++) s = __dadd_rn(s, part[16 * j + i]);
    tot[j] = s;
  }
  __syncthreads();
}

// Router row `row` (row E: the shared gate) against tokens t0 .. t0 + nt - 1 of x (written in this launch with kHc).
template <bool kHc>
__device__ __forceinline__ void router_dot(const DecodeParams &p, uint32_t row, uint32_t t0, uint32_t nt, double *part,
                                           double *tot) {
  bf16_dot<kHc>(p.router + (uint64_t)row * p.H, p.x, p.H, p.H, t0, nt, part, tot);
}

// ---------------------------------------------------------------------------------------------------------------
// Hyper-connection items (the mix before the block; its combine is in combine_item)

// A double summed over the work-group in a fixed order (each wave's lanes by halving exchanges, then the four waves
// in order); every thread receives it. red: 4 doubles of LDS.
__device__ __forceinline__ double wg_sum_f64(double v, double *red) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = __dadd_rn(v, __shfl_xor(v, o, 64));
  __syncthreads();
  if (lane_id() == 0) red[wave_id()] = v;
  __syncthreads();
  return __dadd_rn(__dadd_rn(red[0], red[1]), __dadd_rn(red[2], red[3]));
}

// The norm items' scales (T x 4 fp32), in the hc_n buffer after bf16(n) (T x 4 H bf16).
__device__ __forceinline__ float *hc_scale(const DecodeParams &p) {
  return (float *)((uint16_t *)p.hc_n + (uint64_t)p.T * kHcStreams * p.H);
}

// Norm item (t, s): stream s of token t as RMSNorm(R_s) gamma_s (MODEL_LAYER.md 1.1 step 1; ggml_compute_forward_
// rms_norm_f32: the squares summed in double, mean = sum / H rounded to fp32, scale = 1 / sqrtf(mean + 1e-6), then
// (R scale) gamma), stored for the down and up items.
__device__ __forceinline__ void hc_norm_item(const DecodeParams &p, uint32_t t, uint32_t s, double *red) {
  const uint32_t H = p.H;
  const float *R = p.hc_R + ((uint64_t)t * kHcStreams + s) * H;
  double ss = 0.0;
  for (uint32_t i = tid(); i < H; i += kWG) {
    const float v = R[i];
    ss = __dadd_rn(ss, (double)__fmul_rn(v, v));
  }
  ss = wg_sum_f64(ss, red);
  const float mean = (float)(ss / (double)H);
  // sqrtf is the correctly rounded square root here (__fsqrt_rn is the hardware approximation in this build).
  const float scale = __fdiv_rn(1.0f, sqrtf(__fadd_rn(mean, 1e-6f)));
  // bf16(n), eight values a thread and 16-byte piece written through to the coherence point in one request (the
  // down items' operand); the scale (the up items form n in fp32 again from R, the scale and gamma).
  uint16_t *nb = (uint16_t *)p.hc_n + (uint64_t)t * kHcStreams * H;
  for (uint32_t i = 8 * tid(); i < H; i += 8 * kWG) {
    uint32_t o[4];
#pragma unroll
    for (uint32_t h = 0; h < 2; h++) {
      const float4 r = *(const float4 *)(R + i + 4 * h), g = *(const float4 *)(p.hc_gamma + s * H + i + 4 * h);
      float b0, b1, b2, b3;
      round_bf16_2(__fmul_rn(__fmul_rn(r.x, scale), g.x), __fmul_rn(__fmul_rn(r.y, scale), g.y), b0, b1);
      round_bf16_2(__fmul_rn(__fmul_rn(r.z, scale), g.z), __fmul_rn(__fmul_rn(r.w, scale), g.w), b2, b3);
      o[2 * h] = (__float_as_uint(b0) >> 16) | (__float_as_uint(b1) & 0xffff0000u);
      o[2 * h + 1] = (__float_as_uint(b2) >> 16) | (__float_as_uint(b3) & 0xffff0000u);
    }
    st_co16(nb, (s * H + i) * 2, make_uint4(o[0], o[1], o[2], o[3]));
  }
  if (tid() == 0) st_co(hc_scale(p) + kHcStreams * t + s, scale);
  set_flag(p, kFlagHcNorm + kHcStreams * t + s);
}

// Down item r (after every norm item): row r of W_down (r < lr) or of W_inject (r - lr) against bf16(n) of every
// token, in fp64 as the router's rows; W_down's rows become silu(v / 4) (1.1 step 2), the inject rows stay logits
// (step 4). The last down item in raises kFlagHcDown.
__device__ __forceinline__ void hc_down_item(const DecodeParams &p, uint32_t r, double *part, double *tot,
                                             const uint64_t *tab, uint32_t *s_flag) {
  const uint32_t K = kHcStreams * p.H, lr = p.hc_lr;
  wait_flags(p, kFlagHcNorm, kHcStreams * p.T);
  const uint16_t *W = r < lr ? p.hc_down + (uint64_t)r * K : p.hc_inj + (uint64_t)(r - lr) * K;
  bf16_dot<true, true>(W, p.hc_n, K, K, 0, p.T, part, tot);
  const uint32_t t = tid();
  if (t < p.T) {
    const float v = (float)tot[t];
    float o = v;
    if (r < lr) {  // silu(v / 4): the quarter is exact; silu(z) = z / (1 + e^-z)
      const float z = __fmul_rn(v, 0.25f);
      o = __fdiv_rn(z, __fadd_rn(1.0f, expf_libm(-z, tab)));
    }
    st_co(p.hc_l + (uint64_t)t * (lr + kHcStreams) + r, o);
  }
  if (arrive_last(p.cnt_hc, lr + kHcStreams, s_flag)) set_flag(p, kFlagHcDown);
}

// Up item j (after the down items): values i = kHcUpValues j .. + kHcUpValues - 1 of x. Rows s H + i of W_up (one a
// quarter of the threads, the tokens dealt to the four threads of a row) against bf16(l) of every token in fp64,
// k ascending; then x[i] = (sum over s in order of n_s[i] sigma(a_s[i])) / 4 (1.1 step 3). The last up item in raises
// kFlagHcX.
__device__ __forceinline__ void hc_up_item(const DecodeParams &p, uint32_t j, uint8_t *lds, const uint64_t *tab,
                                           uint32_t *s_flag) {
  const uint32_t H = p.H, T = p.T, lr = p.hc_lr, lw = lr + kHcStreams, i0 = kHcUpValues * j;
  wait_flag(p, kFlagHcDown);
  float *lb = (float *)lds;                                   // [t][k] bf16(l) as floats
  float *a = lb + T * lr;                                     // [t][s][i - i0]
  for (uint32_t e = tid(); e < T * lr; e += kWG) lb[e] = round_bf16(ld_co(p.hc_l + (uint64_t)(e / lr) * lw + e % lr));
  __syncthreads();
  {
    const uint32_t rr = tid() / 4, q = tid() % 4;  // row rr of the item's 4 kHcUpValues (64), token group q
    const uint32_t s = rr / kHcUpValues, i = i0 + rr % kHcUpValues;
    const uint16_t *W = p.hc_up + ((uint64_t)s * H + i) * lr;
    // The row's weights 32 values at a time (four loads issued together, shared by the thread's tokens), each token's
    // chain continuing through them in k order.
    double acc[kMaxDecodeTokens / 4] = {};
    for (uint32_t k0 = 0; k0 < lr; k0 += 32) {
      uint4 w[4];
#pragma unroll
      for (uint32_t j = 0; j < 4; j++) w[j] = k0 + 8 * j < lr ? *(const uint4 *)(W + k0 + 8 * j) : make_uint4(0u, 0u, 0u, 0u);
#pragma unroll
      for (uint32_t tt = 0; tt < kMaxDecodeTokens / 4; tt++) {
        const uint32_t t = q + 4 * tt;
        if (t >= T) break;
#pragma unroll
        for (uint32_t j = 0; j < 4; j++) {
          if (k0 + 8 * j >= lr) break;
          const uint32_t wv[4] = {w[j].x, w[j].y, w[j].z, w[j].w};
#pragma unroll
          for (int m = 0; m < 8; m++) {
            const float wf = __uint_as_float((m & 1) ? wv[m / 2] & 0xffff0000u : wv[m / 2] << 16);
            acc[tt] = __builtin_fma((double)wf, (double)lb[t * lr + k0 + 8 * j + m], acc[tt]);
          }
        }
      }
    }
#pragma unroll
    for (uint32_t tt = 0; tt < kMaxDecodeTokens / 4; tt++) {
      const uint32_t t = q + 4 * tt;
      if (t < T) a[(t * kHcStreams + s) * kHcUpValues + rr % kHcUpValues] = (float)acc[tt];
    }
  }
  __syncthreads();
  {
    const uint32_t t = tid() / kHcUpValues, di = tid() % kHcUpValues, i = i0 + di;
    if (t < T) {
      float acc = 0.0f;
#pragma unroll
      for (uint32_t s = 0; s < kHcStreams; s++) {
        const float n = __fmul_rn(__fmul_rn(p.hc_R[((uint64_t)t * kHcStreams + s) * H + i],
                                            ld_co(hc_scale(p) + kHcStreams * t + s)), p.hc_gamma[s * H + i]);
        acc = __fadd_rn(acc, __fmul_rn(n, sigmoid_libm(a[(t * kHcStreams + s) * kHcUpValues + di], tab)));
      }
      st_co(p.hc_x + (uint64_t)t * H + i, __fmul_rn(acc, 0.25f));
    }
  }
  if (arrive_last(p.cnt_hc + kDynStride, H / kHcUpValues, s_flag)) set_flag(p, kFlagHcX);
}

// Router rows row0 .. row0 + nr - 1 (nr <= kRouteRows) against every token, rounded to fp32 and stored as the
// logits' tagged records (the top-k item adds the bias). Each row's arithmetic is bf16_dot's (the same k chains a lane, the same 16-lane tree, the same
// chunk and partial order), so a logit does not depend on kRouteRows; x is read once for the rows (a lane holds its
// eight values of eight tokens), which divides the device's reads of x by kRouteRows. part: kRouterLds of LDS.
template <bool kHc>
__device__ __forceinline__ void router_rows(const DecodeParams &p, uint32_t row0, uint32_t nr, double *part) {
  const uint32_t lane = lane_id(), wv = wave_id(), K = p.H, nC = K / 512, T = p.T;
  const uint32_t pslot = 4 * wv + lane / 16;
  const uint16_t *W = p.router + (uint64_t)row0 * K;
  for (uint32_t c = wv; c < nC; c += kWG / 64) {
    uint4 wa[kRouteRows];
#pragma unroll
    for (uint32_t r = 0; r < kRouteRows; r++)
      wa[r] = *(const uint4 *)(W + (uint64_t)min(r, nr - 1) * K + 512 * c + 8 * lane);
    for (uint32_t tb = 0; tb < T; tb += 8) {
      const uint32_t nb = min(8u, T - tb);
      float xs[8][8];  // token tb + tt's eight values, rounded to bf16
#pragma unroll
      for (uint32_t tt = 0; tt < 8; tt++) {
        const uint64_t e = (uint64_t)(tb + min(tt, nb - 1)) * K + 512 * c + 8 * lane;
        float4 xa, xb;
        if constexpr (kHc) {
          const uint4 u = ld_co16(p.x, (uint32_t)(4 * e)), v = ld_co16(p.x, (uint32_t)(4 * e + 16));
          xa = make_float4(__uint_as_float(u.x), __uint_as_float(u.y), __uint_as_float(u.z), __uint_as_float(u.w));
          xb = make_float4(__uint_as_float(v.x), __uint_as_float(v.y), __uint_as_float(v.z), __uint_as_float(v.w));
        } else {
          xa = ((const float4 *)(p.x + e))[0], xb = ((const float4 *)(p.x + e))[1];
        }
        round_bf16_2(xa.x, xa.y, xs[tt][0], xs[tt][1]), round_bf16_2(xa.z, xa.w, xs[tt][2], xs[tt][3]);
        round_bf16_2(xb.x, xb.y, xs[tt][4], xs[tt][5]), round_bf16_2(xb.z, xb.w, xs[tt][6], xs[tt][7]);
      }
#pragma unroll
      for (uint32_t r = 0; r < kRouteRows; r++) {
        if (r >= nr) break;
        __builtin_amdgcn_sched_barrier(0);  // one row's chains at a time (registers)
        double wd[8];
        const uint32_t w0[4] = {wa[r].x, wa[r].y, wa[r].z, wa[r].w};
#pragma unroll
        for (int k = 0; k < 8; k++) wd[k] = (double)__uint_as_float((k & 1) ? w0[k / 2] & 0xffff0000u : w0[k / 2] << 16);
        double v[8];
#pragma unroll
        for (uint32_t tt = 0; tt < 8; tt++) {
          double a = 0.0;
          if (tt < nb) {
#pragma unroll
            for (int k = 0; k < 8; k++) a = __builtin_fma(wd[k], (double)xs[tt][k], a);
          }
          v[tt] = a;
        }
        const double s = row16_reduce8_f64(v);  // bf16_dot's tree
        const uint32_t tt = (lane & 15u) / 2;
        if ((lane & 1u) == 0 && tt < nb) {
          double *q = part + ((r * kMaxDecodeTokens) + tb + tt) * 16 + pslot;
          *q = c == wv ? s : __dadd_rn(*q, s);
        }
      }
    }
  }
  if (wv >= nC && (lane & 15u) == 0) {  // waves without a chunk (K < 2048) give zeros
    for (uint32_t r = 0; r < nr; r++)
      for (uint32_t t = 0; t < T; t++) part[((r * kMaxDecodeTokens) + t) * 16 + pslot] = 0.0;
  }
  __syncthreads();
  const uint32_t oi = tid(), orow = oi / T;  // the thread's output: row orow, token oi % T
  if (orow < nr) {
    const uint32_t t = oi % T;
    double s = 0.0;
#pragma unroll
    for (uint32_t i = 0; i < 16; i++) s = __dadd_rn(s, part[((orow * kMaxDecodeTokens) + t) * 16 + i]);
    st_tag(p.logits + (uint64_t)t * (p.E + 1) + row0 + orow, __float_as_uint((float)s), p.tag);
  }
  __syncthreads();
}

// ---------------------------------------------------------------------------------------------------------------
// Groups

// The launch's groups, in LDS: each work-group builds the table itself from the routed ids (the same table in every
// work-group), or copies a pre-routed call's from the host's.
struct GroupTab {
  uint32_t ng;
  int32_t slot[kMaxGroups];
  uint32_t n[kMaxGroups];
  uint16_t asg[kMaxGroups][MOE_GROUP_MAX];
};

// MoeGroup records from the routed ids: an expert's assignments in order, MOE_GROUP_MAX a group (as group_slots,
// layer.cl:894-942); numbered by decreasing size, then by first assignment. An expert takes at most one assignment a
// token, so a mask of the tokens that chose it gives each assignment its rank among the expert's (and whether it heads
// a group). A head's number is the count of heads of larger groups plus those of its size at lower assignments: a
// ballot per size and wave gives both. Only the ids are read here (every work-group reads them, so the fewer lines the
// better); the combine reads the weights.
__device__ __forceinline__ void make_groups(const DecodeParams &p, uint8_t *lds, GroupTab *tab) {
  const uint32_t T = p.T, K = p.K, E = p.E, n = T * K, a = tid(), lane = lane_id(), wv = wave_id();
  uint32_t *ids = (uint32_t *)lds, *mask = ids + kMaxDecodeTokens * kMaxUsed, *gnum = mask + kMaxExperts;
  uint32_t *cnt = gnum + 2 * kMaxExperts;  // [wave][size 1 .. MOE_GROUP_MAX]
  for (uint32_t i = a; i < E; i += kWG) mask[i] = 0u;
  const uint32_t t = a / K;
  // Each id's reader polls its own record (at most kMaxDecodeTokens kMaxUsed a work-group, ten cache lines at T = 8).
  if (a < n) {
    uint64_t ri;
    for (uint32_t k = 0;; k++) {
      ri = ld_tag(p.ids_t + a);
      if (tag_of(ri) == p.tag) break;
      __builtin_amdgcn_s_sleep(C0VEN_POLL_SLEEP);
      if (k == kSpinLimit) {
        st_co(p.err, 1u);
        break;
      }
    }
    ids[a] = (uint32_t)ri;
  }
  __syncthreads();
  // Assignments to experts not on the device (misses) join no group.
  const bool live = a < n && (!p.resident || p.resident[ids[a]]);
  if (T == 1) {  // one token: every group is one assignment, in rank order (what the general numbering gives)
    const uint64_t b = __ballot(live);  // a < K < 64: wave 0 holds them all
    if (wv == 0 && live) {
      const uint32_t g = __builtin_amdgcn_mbcnt_lo((uint32_t)b, 0u);
      tab->slot[g] = (int32_t)ids[a];
      tab->n[g] = 1u;
      tab->asg[g][0] = (uint16_t)a;
    }
    if (a == 0) tab->ng = (uint32_t)__popcll(b);
    __syncthreads();
    return;
  }
  uint32_t e = 0, rank = 0, total = 0;
  if (live) {
    e = ids[a];
    atomicOr(mask + e, 1u << t);
  }
  __syncthreads();
  if (live) {
    const uint32_t m = mask[e];
    rank = __popc(m & ((1u << t) - 1u));
    total = __popc(m);
  }
  const bool head = live && rank % MOE_GROUP_MAX == 0;
  const uint32_t gn = head ? min((uint32_t)MOE_GROUP_MAX, total - rank) : 0u;
  uint32_t before = 0;  // heads of this size at lower assignments of this wave
#pragma unroll
  for (uint32_t sz = 1; sz <= MOE_GROUP_MAX; sz++) {
    const uint64_t b = __ballot(gn == sz);
    if (gn == sz) before = __builtin_amdgcn_mbcnt_hi((uint32_t)(b >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)b, 0u));
    if (lane == 0) cnt[wv * MOE_GROUP_MAX + sz - 1] = (uint32_t)__popcll(b);
  }
  __syncthreads();
  uint32_t g = before, G = 0;
#pragma unroll
  for (uint32_t w = 0; w < kWG / 64; w++)
#pragma unroll
    for (uint32_t sz = 1; sz <= MOE_GROUP_MAX; sz++) {
      const uint32_t c = cnt[w * MOE_GROUP_MAX + sz - 1];
      G += c;
      g += (sz > gn || (sz == gn && w < wv)) ? c : 0u;
    }
  if (head) {
    gnum[2 * e + rank / MOE_GROUP_MAX] = g;
    tab->slot[g] = (int32_t)e;
    tab->n[g] = gn;
  }
  __syncthreads();
  if (live) tab->asg[gnum[2 * e + rank / MOE_GROUP_MAX]][rank % MOE_GROUP_MAX] = (uint16_t)a;
  if (a == 0) tab->ng = G;
  __syncthreads();
}

// A pre-routed call's groups (written by the host before the launch) into the table.
__device__ __forceinline__ void copy_groups(const DecodeParams &p, GroupTab *tab) {
  const uint32_t ng = *p.ngroups;
  for (uint32_t g = tid(); g < ng; g += kWG) {
    const MoeGroup m = p.groups[g];
    tab->slot[g] = m.slot;
    tab->n[g] = m.n;
#pragma unroll
    for (uint32_t j = 0; j < MOE_GROUP_MAX; j++) tab->asg[g][j] = (uint16_t)m.asg[j];
  }
  if (tid() == 0) tab->ng = ng;
  __syncthreads();
}

// ---------------------------------------------------------------------------------------------------------------
// Expert items

struct GroupLds {
  int32_t slot;
  uint32_t n, gid, asg[MOE_GROUP_MAX], tok[MOE_GROUP_MAX];
};

__device__ __forceinline__ uint32_t asg_token(const DecodeParams &p, uint32_t asg) {
  const uint32_t n = p.T * p.K;
  return asg < n ? asg / p.K : asg - n;
}

// Group g of the table (gid g), or the shared expert's token chunk c (gid T K + c: assignments T K + 8 c + j).
__device__ __forceinline__ void read_group(const DecodeParams &p, const GroupTab *tab, bool shared, uint32_t g,
                                           GroupLds *s) {
  if (tid() == 0) {
    if (shared) {
      s->slot = (int32_t)p.E, s->n = min((uint32_t)MOE_GROUP_MAX, p.T - MOE_GROUP_MAX * g), s->gid = p.T * p.K + g;
    } else {
      s->slot = tab->slot[g], s->n = tab->n[g], s->gid = g;
    }
  }
  if (tid() < MOE_GROUP_MAX) {
    const uint32_t a = shared ? p.T * p.K + MOE_GROUP_MAX * g + tid() : tab->asg[g][tid()];
    s->asg[tid()] = a;
    s->tok[tid()] = asg_token(p, a);
  }
  __syncthreads();
}

// Activation units (act + unit index * kActBytes, coherent) of the group's assignments into LDS: unit (j, u) at
// j act_tok_stride(U) + u kActLds.
__device__ __forceinline__ void stage_act(const uint8_t *act, const uint32_t *unit_of_j, uint32_t n, uint32_t U,
                                          uint8_t *lds) {
  // Eight loads of a thread in flight before their stores (one round trip a batch, not one a chunk).
  constexpr uint32_t kBatch = 8;
  const uint32_t total = n * U * (kActBytes / 16);
  for (uint32_t i0 = 0; i0 < total; i0 += kBatch * kWG) {
    uint4 v[kBatch];
#pragma unroll
    for (uint32_t k = 0; k < kBatch; k++) {
      const uint32_t i = min(i0 + k * kWG + tid(), total - 1);
      const uint32_t unit = i / (kActBytes / 16), c = i % (kActBytes / 16), j = unit / U, u = unit % U;
      v[k] = ld_co16(act, (unit_of_j[j] * U + u) * kActBytes + 16 * c);
    }
#pragma unroll
    for (uint32_t k = 0; k < kBatch; k++) {
      const uint32_t i = i0 + k * kWG + tid();
      if (i < total) {
        const uint32_t unit = i / (kActBytes / 16), c = i % (kActBytes / 16), j = unit / U, u = unit % U;
        *(uint4 *)(lds + j * act_tok_stride(U) + u * kActLds + 16 * c) = v[k];
      }
    }
  }
}

// h of the group's assignments quantised to the down's activation type straight into LDS: unit (j, u) at
// j act_tok_stride(U) + u kActLds, a half-wave a unit. The values are polled as tagged records (the gate/up items'
// stores are the hand-off), two records a 16-byte load. Every down item of the group quantises the same h the same way.
__device__ __forceinline__ void stage_h(const DecodeParams &p, const GroupLds *sg, uint32_t dact, uint32_t U,
                                        uint8_t *lds) {
  const uint32_t l32 = tid() & 31u;
  wait_tag(p, p.h + (uint64_t)sg->asg[sg->n - 1] * p.F + p.F - 1);  // one record first, then all
  for (uint32_t i = tid() / 32; i < sg->n * U; i += kWG / 32) {
    const uint32_t j = i / U, u = i % U;
    const uint32_t off = (sg->asg[j] * p.F + u * kUnit + 8 * l32) * (uint32_t)sizeof(uint64_t);
    uint64_t r[8];
    if (u * kUnit + 8 * l32 >= p.F) {  // past the row's end (a partial last unit): zeros
#pragma unroll
      for (int k = 0; k < 8; k++) r[k] = 0;
    } else
    for (uint32_t n = 0;; n++) {
      bool ok = true;
#pragma unroll
      for (int k = 0; k < 4; k++) {
        const uint4 v = ld_co16(p.h, off + 16 * k);
        r[2 * k] = ((uint64_t)v.y << 32) | v.x, r[2 * k + 1] = ((uint64_t)v.w << 32) | v.z;
      }
#pragma unroll
      for (int k = 0; k < 8; k++) ok &= tag_of(r[k]) == p.tag;
      if (ok) break;
      __builtin_amdgcn_s_sleep(C0VEN_POLL_SLEEP);
      if (n == kSpinLimit) {
        st_co(p.err, 1u);
        break;
      }
    }
    float v[8];
#pragma unroll
    for (int k = 0; k < 8; k++) v[k] = __uint_as_float((uint32_t)r[k]);
    quant_unit<true>(v, l32, dact, lds + j * act_tok_stride(U) + u * kActLds);
  }
}

// The q8_K units in LDS (n tokens x U) get their block sums split for the matrix cores' minimum part, once for the
// work-group (ActB::put_split), instead of once per wave and unit.
__device__ __forceinline__ void presplit(uint32_t n, uint32_t U, uint8_t *lds) {
  if (tid() < n * U) ActB::put_split(lds + (tid() / U) * act_tok_stride(U) + (tid() % U) * kActLds);
  __syncthreads();
}

// Groups of at least this many tokens take the matrix-core paths (Q4_K weights, 8 units a gate/up row, 2 a down row);
// smaller ones the dot4 paths, where the 16 token columns of an MFMA would be mostly padding.
constexpr uint32_t kMfmaMinTokens = 3;

template <uint32_t kTypes>
__device__ __forceinline__ bool use_mfma(uint32_t type, uint32_t U, uint32_t U_mfma, uint32_t n) {
  return (kTypes & kTypeQ4_K) != 0 && type == QT_Q4_K && U == U_mfma && n >= kMfmaMinTokens;
}

// Gate and up of rows 16 blk .. 16 blk + 15 on the matrix cores (U = 8). Wave w takes matrix w & 1 and units
// 4 (w >> 1) .. + 3 of the 16 rows for all tokens (q4k_terms); the second half's unit terms go through LDS (xch) to
// the first, which adds them to its sums in unit order (0 + t_0 + t_1 ...: the oracle's sequence). The gate and up
// sums then go through LDS and each thread takes one (row, token): h = swiglu, stored as a tagged record.
__device__ __forceinline__ void gate_up_mfma(const DecodeParams &p, const GroupLds *sg, const GroupMat &gm, uint32_t blk,
                                             uint8_t *lds, float *xch, const uint64_t *tab, uint64_t *mark) {
  constexpr uint32_t U = 8;
  const uint32_t lane = lane_id(), w = wave_id(), m = w & 1u, half = w >> 1, n = sg->n, row0 = 16 * blk;
  const uint8_t *mat = gm.mat + (m ? (gm.shared ? p.sh_up_off : p.ex_up_off) : 0);
  Q4kRaw raw[4];  // all four units' weights in flight before the activations are waited for
#pragma unroll
  for (uint32_t k = 0; k < 4; k++) raw[k].load(mat, U, row0, 4 * half + k, lane);
  if (gm.shared && p.route) wait_flags(p, kFlagLead + sg->tok[0], n);
  stage_act(gm.shared ? p.act_s : p.act_r, sg->tok, n, U, lds);
  __syncthreads();
  presplit(n, U, lds);
  if (mark && tid() == 0) mark[1] = __builtin_amdgcn_s_memrealtime();
  const uint32_t j = min(lane % 16, n - 1);
  float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
  for (uint32_t k = 0; k < 4; k++) {
    const uint32_t u = 4 * half + k;
    Q4kA a;
    a.decode(raw[k], lane);
    ActB b;
    b.load_presplit(lds + j * act_tok_stride(U) + u * kActLds, lane);
    float t[4];
    q4k_terms(a, b, t);
#pragma unroll
    for (uint32_t i = 0; i < 4; i++) {
      if (half == 0) {
        acc[i] = __fadd_rn(acc[i], t[i]);
      } else {
        xch[((m * 4 + k) * 4 + i) * 64 + lane] = t[i];
      }
    }
  }
  __syncthreads();
  float *sums = xch + 2 * 4 * 4 * 64;  // [matrix][row][token]
  if (half == 0) {
#pragma unroll
    for (uint32_t k = 0; k < 4; k++)
#pragma unroll
      for (uint32_t i = 0; i < 4; i++) acc[i] = __fadd_rn(acc[i], xch[((m * 4 + k) * 4 + i) * 64 + lane]);
#pragma unroll
    for (uint32_t i = 0; i < 4; i++) sums[(m * 16 + 4 * (lane / 16) + i) * 16 + lane % 16] = acc[i];
  }
  __syncthreads();
  const uint32_t r = tid() / 16, tok = tid() % 16;
  if (tok < n) {
    const float g = sums[r * 16 + tok], up = sums[(16 + r) * 16 + tok];
    st_tag(p.h + (uint64_t)sg->asg[tok] * p.F + row0 + r, __float_as_uint(swiglu_one(g, up, p.swiglu_limit, tab)), p.tag);
  }
  if (mark && tid() == 0) mark[2] = __builtin_amdgcn_s_memrealtime();
}

// Down rows 128 blk .. 128 blk + 127 on the matrix cores (U = 2): wave w takes rows 32 w .. + 31 as two 16-row tiles,
// both units in order; each lane stores its rows 4 g + i of token l % 16.
__device__ __forceinline__ void down_mfma(const DecodeParams &p, const GroupLds *sg, const GroupMat &gm, uint32_t blk,
                                          uint8_t *lds, uint64_t *mark) {
  constexpr uint32_t U = 2;
  const uint32_t lane = lane_id(), n = sg->n, row0 = 128 * blk + 32 * wave_id();
  Q4kRaw raw[2][U];  // every tile-unit's weights in flight before h is waited for
#pragma unroll
  for (uint32_t tt = 0; tt < 2; tt++)
#pragma unroll
    for (uint32_t u = 0; u < U; u++) raw[tt][u].load(gm.mat, U, row0 + 16 * tt, u, lane);
  stage_h(p, sg, QT_Q8_K, U, lds);
  __syncthreads();
  presplit(n, U, lds);
  if (mark && tid() == 0) mark[1] = __builtin_amdgcn_s_memrealtime();
  const uint32_t j = min(lane % 16, n - 1);
  float acc[2][4] = {{0.0f, 0.0f, 0.0f, 0.0f}, {0.0f, 0.0f, 0.0f, 0.0f}};
#pragma unroll
  for (uint32_t u = 0; u < U; u++) {
    ActB b;
    b.load_presplit(lds + j * act_tok_stride(U) + u * kActLds, lane);
#pragma unroll
    for (uint32_t tt = 0; tt < 2; tt++) {
      Q4kA a;
      a.decode(raw[tt][u], lane);
      float t[4];
      q4k_terms(a, b, t);
#pragma unroll
      for (uint32_t i = 0; i < 4; i++) acc[tt][i] = __fadd_rn(acc[tt][i], t[i]);
    }
  }
  const uint32_t tok = lane % 16;
  if (tok < n) {
    uint64_t *dst = p.y_asg + (uint64_t)sg->asg[tok] * p.H + row0 + 4 * (lane / 16);
#pragma unroll
    for (uint32_t tt = 0; tt < 2; tt++)
#pragma unroll
      for (uint32_t i = 0; i < 4; i++) st_tag(dst + 16 * tt + i, __float_as_uint(acc[tt][i]), p.tag);
  }
  if (mark && tid() == 0) mark[2] = __builtin_amdgcn_s_memrealtime();
}

// Gate and up of rows blk * gate_up_rows .. of the group: wave w takes matrix w % 2 and rows (w / 2) 64 / U .. (lane
// r U + u), so that a load of one piece reads 64 / U consecutive rows of each unit (a whole line at U = 8); the up waves
// hand their row sums to the gate waves through LDS, which store h = silu(g) * u per row as tagged records.
template <uint32_t kTypes>
__device__ __forceinline__ void gate_up_item(const DecodeParams &p, const GroupLds *sg, uint32_t blk, uint8_t *lds,
                                             uint32_t *grid_lds, uint32_t *grid_have, const uint64_t *tab,
                                             uint64_t *mark) {
  // U units a row, UL lanes a row (U rounded up to a power of two; lanes past U add exact zeros).
  const uint32_t U = units_of(p.H), UL = unit_lanes(U), rows = gate_up_rows(UL), row0 = blk * rows, n = sg->n;
  const GroupMat gm0 = group_mat(p, sg->slot, 0);
  // Gate and up share a type except for a shared expert whose matrices differ (both then codebook-free).
  if (use_mfma<kTypes>(gm0.type, U, 8, n) && (!gm0.shared || p.sh_up_type == gm0.type)) {
    gate_up_mfma(p, sg, gm0, blk, lds, (float *)(lds + MOE_GROUP_MAX * act_tok_stride(U)), tab, mark);
    return;
  }
  if ((kTypes & (kTypeIQ3_S | kTypeIQ2)) && grid_family(gm0.type)) load_grid(p, gm0.type, grid_lds, grid_have);
  const uint32_t lane = lane_id(), m = wave_id() & 1u, r = lane / UL, u = lane % UL, ue = u < U ? u : 0u;
  const uint32_t rl = (wave_id() >> 1) * (64 / UL) + r, row = row0 + rl;  // rl: the row within the item
  const GroupMat gm = m ? group_mat(p, sg->slot, 1) : gm0;  // this wave's matrix (wave-uniform)
  const uint8_t *mat = gm.mat;
  const uint8_t *tile = mat + (uint64_t)(row / kTileRows) * tile_bytes(gm.type, U);
  float t[MOE_GROUP_MAX];
  pair_terms<kTypes>(gm.type, tile, pair_idx(row % kTileRows, ue), kTileRows * U, grid_lds,
             (const uint32_t *)lds + ue * (kActLds / 4), act_tok_stride(U) / 4, n, t, [&] {
               // The shared expert's items run beside the router: x of their tokens is quantised by lead items
               // 8 c .. (their flags); routed groups exist only once every lead item is in.
               if (gm.shared && p.route) wait_flags(p, kFlagLead + sg->tok[0], n);
               stage_act(gm.shared ? p.act_s : p.act_r, sg->tok, n, U, lds);
               __syncthreads();
               if (mark && tid() == 0) mark[1] = __builtin_amdgcn_s_memrealtime();
             });
  float *xs = (float *)(lds + MOE_GROUP_MAX * act_tok_stride(U));  // up's row sums [row in item][token]
#pragma unroll
  for (uint32_t j = 0; j < MOE_GROUP_MAX; j++) {
    if (j >= n) break;
    t[j] = row_sum(u < U ? t[j] : 0.0f, UL);  // the row's sum in every lane of the row
    if (m == 1 && u == 0) xs[rl * MOE_GROUP_MAX + j] = t[j];
  }
  __syncthreads();
  if (m == 0 && u == 0) {
#pragma unroll
    for (uint32_t j = 0; j < MOE_GROUP_MAX; j++) {
      if (j >= n) break;
      st_tag(p.h + (uint64_t)sg->asg[j] * p.F + row,
             __float_as_uint(swiglu_one(t[j], xs[rl * MOE_GROUP_MAX + j], p.swiglu_limit, tab)), p.tag);
    }
  }
  if (mark && tid() == 0) mark[2] = __builtin_amdgcn_s_memrealtime();
}

// Down rows blk * down_rows .. of the group (lane = r * U + u), then the combine of every token this item completes.
template <uint32_t kTypes>
__device__ __forceinline__ void down_item(const DecodeParams &p, const GroupLds *sg, uint32_t blk, uint8_t *lds,
                                          uint32_t *grid_lds, uint32_t *grid_have, uint64_t *mark) {
  const uint32_t U = units_of(p.F), UL = unit_lanes(U), rows = down_rows(UL), row0 = blk * rows, n = sg->n;
  const GroupMat gm = group_mat(p, sg->slot, 2);
  if (use_mfma<kTypes>(gm.type, U, 2, n) && p.F == 2 * kUnit) {
    down_mfma(p, sg, gm, blk, lds, mark);
  } else {
    if ((kTypes & (kTypeIQ3_S | kTypeIQ2)) && grid_family(gm.type)) load_grid(p, gm.type, grid_lds, grid_have);
    const uint32_t lane = lane_id(), r = lane / UL, u = lane % UL, ue = u < U ? u : 0u;
    const uint32_t row = row0 + wave_id() * (64 / UL) + r;
    const uint8_t *tile = gm.mat + (uint64_t)(row / kTileRows) * tile_bytes(gm.type, U);
    float t[MOE_GROUP_MAX];
    pair_terms<kTypes>(gm.type, tile, pair_idx(row % kTileRows, ue), kTileRows * U, grid_lds,
               (const uint32_t *)lds + ue * (kActLds / 4), act_tok_stride(U) / 4, n, t, [&] {
                 stage_h(p, sg, act_type<kTypes>(quant_vec_dot_type(gm.type)), U, lds);
                 __syncthreads();
                 if (mark && tid() == 0) mark[1] = __builtin_amdgcn_s_memrealtime();
               });
#pragma unroll
    for (uint32_t j = 0; j < MOE_GROUP_MAX; j++) {
      if (j >= n) break;
      const float s = row_sum(u < U ? t[j] : 0.0f, UL);
      if (u == 0) st_tag(p.y_asg + (uint64_t)sg->asg[j] * p.H + row, __float_as_uint(s), p.tag);
    }
    if (mark && tid() == 0) mark[2] = __builtin_amdgcn_s_memrealtime();
  }
}

// Combine item (token t, rows blk * down_rows ..): y = sum_k w_k y_k in rank order, then + gs s, a row a thread. The
// token's weights (and, for a pre-routed call, which of its assignments are live) are read once into LDS; the
// per-assignment outputs are polled as tagged records (one first, then all of the row's). The combine items come after
// every down item, so what they wait for has a smaller number.
template <bool kHc>
__device__ __forceinline__ void combine_item(const DecodeParams &p, uint32_t t, uint32_t blk, float *wl,
                                             const uint64_t *tab, uint64_t *mark) {
  const uint32_t rows = down_rows(unit_lanes(units_of(p.F))), K = p.K, row = blk * rows + tid();
  const uint32_t ns = p.has_shared ? 1u : 0u;
  {
    const uint32_t k = tid();
    if (k < K) {  // thread k: w_k and whether assignment k is live (a pre-routed call marks a dead one id < 0, a
                  // routed one is dead when its expert is a miss)
      const float w = p.route ? __uint_as_float(poll_tag(p, p.w_t + t * K + k)) : ld_co(p.w + t * K + k);
      const bool on = p.route ? (!p.resident || p.resident[poll_tag(p, p.ids_t + t * K + k)]) : ld_co(p.ids + t * K + k) >= 0;
      wl[k] = w;
      wl[kMaxUsed + 1 + k] = on ? 1.0f : 0.0f;
    } else if (k == K && ns) {  // thread K: the shared expert's gate
      wl[K] = __uint_as_float(poll_tag(p, p.gs + t));
    } else if (kHc && k >= K + 1 && k < K + 1 + kHcStreams) {  // stream s's weight 2 sigma(inject_s / 4)
      const uint32_t s = k - K - 1;
      const float inj = ld_co(p.hc_l + (uint64_t)t * (p.hc_lr + kHcStreams) + p.hc_lr + s);
      wl[2 * kMaxUsed + 1 + s] = __fmul_rn(2.0f, sigmoid_libm(__fmul_rn(inj, 0.25f), tab));
    }
  }
  if (p.route && !p.resident) wait_tag(p, p.y_asg + ((uint64_t)t * K + K - 1) * p.H + blk * rows + rows - 1);
  else __syncthreads();
  // The host's answer for the token's misses (cpu_wait, layer.cl:849-866): thread 0 polls the step with system-scope
  // acquires, bounded in time (5 s on the 100 MHz clock), the work-group follows.
  bool cpu = false;
  if (p.route && p.resident) {
    uint32_t miss = 0;
    for (uint32_t k = 0; k < K; k++) miss += wl[kMaxUsed + 1 + k] == 0.0f ? 1u : 0u;
    cpu = miss > 0 && p.ans_y;
    if (cpu && tid() == 0) {
      const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
      while (__hip_atomic_load(p.ans_seq, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_SYSTEM) != p.tag) {
        __builtin_amdgcn_s_sleep(8);
        if (__builtin_amdgcn_s_memrealtime() - t0 > 500000000ull) {
          st_co(p.err, 1u);
          break;
        }
      }
    }
    __syncthreads();
  }
  if (mark && tid() == 0) mark[1] = __builtin_amdgcn_s_memrealtime();
  if (tid() < rows) {
    bool on[kMaxUsed];
    float wv[kMaxUsed], yv[kMaxUsed];
#pragma unroll
    for (uint32_t k = 0; k < kMaxUsed; k++) {
      on[k] = k < K && wl[kMaxUsed + 1 + k] != 0.0f;
      wv[k] = k < K ? wl[k] : 0.0f;
    }
    const float gs = ns ? wl[K] : 0.0f;
    // The K (+ shared) outputs of this row: all loads in flight together, polled as a set.
    float ys = 0.0f;
    for (uint32_t n = 0;; n++) {
      bool ok = true;
#pragma unroll
      for (uint32_t k = 0; k < kMaxUsed; k++) {
        const uint64_t r = on[k] ? ld_tag(p.y_asg + ((uint64_t)t * K + k) * p.H + row) : ((uint64_t)p.tag << 32);
        ok &= tag_of(r) == p.tag;
        yv[k] = __uint_as_float((uint32_t)r);
      }
      if (ns) {
        const uint64_t r = ld_tag(p.y_asg + ((uint64_t)p.T * K + t) * p.H + row);
        ok &= tag_of(r) == p.tag;
        ys = __uint_as_float((uint32_t)r);
      }
      if (ok) break;
      __builtin_amdgcn_s_sleep(C0VEN_POLL_SLEEP);
      if (n == kSpinLimit) {
        st_co(p.err, 1u);
        break;
      }
    }
    float acc = 0.0f;
#pragma unroll
    for (uint32_t k = 0; k < kMaxUsed; k++)
      if (on[k]) acc = __fadd_rn(acc, __fmul_rn(wv[k], yv[k]));
    if (ns) acc = __fadd_rn(acc, __fmul_rn(gs, ys));
    if (cpu) acc = __fadd_rn(acc, __hip_atomic_load(p.ans_y + (uint64_t)t * p.H + row, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM));
    if (p.y) p.y[(uint64_t)t * p.H + row] = acc;
    if constexpr (kHc) {  // the combine (MODEL_LAYER.md 1.2): R_s += 2 sigma(inject_s / 4) y
#pragma unroll
      for (uint32_t s = 0; s < kHcStreams; s++) {
        float *r = p.hc_R + ((uint64_t)t * kHcStreams + s) * p.H + row;
        *r = __fadd_rn(*r, __fmul_rn(wl[2 * kMaxUsed + 1 + s], acc));
      }
    }
  }
  if (mark && tid() == 0) mark[2] = __builtin_amdgcn_s_memrealtime();
}

}  // namespace

// Grid: the work-groups of 256 the device holds at once; dynamic LDS: the larger of a group's activation units
// (MOE_GROUP_MAX x act_tok_stride) and the grouping's tables (kGroupingLds).
template <uint32_t kTypes, bool kHc>
__global__ void __launch_bounds__(kWG) __attribute__((amdgpu_waves_per_eu(3))) moe_decode(DecodeParams p) {
  extern __shared__ __align__(16) uint8_t lds[];
  __shared__ uint32_t grid_lds[(kTypes & kTypeIQ2) ? kGridWords : (kTypes & kTypeIQ3_S) ? 512 : 1];
  __shared__ uint32_t s_grid;  // the grid type whose codebook grid_lds holds
  __shared__ uint32_t s_flag;
  // A combine item's weights (and gs), which assignments are live, and the streams' weights 2 sigma(inject / 4).
  __shared__ float s_wl[2 * kMaxUsed + 1 + kHcStreams];
  __shared__ double s_part[kMaxDecodeTokens * 16], s_tot[kMaxDecodeTokens];
  __shared__ GroupLds sg;
  __shared__ GroupTab gtab;
  __shared__ uint64_t exp_tab[32];  // expf's table, read at LDS latency
  if (tid() < 32) exp_tab[tid()] = kExp2Tab[tid()];
  if (tid() == 0) s_grid = 0xffffffffu;
  __syncthreads();
  const uint32_t T = p.T, E = p.E, Ug = unit_lanes(units_of(p.H)), Ud = unit_lanes(units_of(p.F));
  const uint32_t nH = kHc ? hc_items(T, p.H, p.hc_lr) : 0u;  // the hyper-connection mix's items come first
  const uint32_t nL = lead_items(T, E, p.route), nTop = p.route ? T : 0, B1 = nH + nL + nTop;
  const uint32_t nGU = p.F / gate_up_rows(Ug), nD = p.H / down_rows(Ud), nBlk = nD;  // combine items: T x nBlk
  const uint32_t ns = shared_chunks(T, p.route, p.has_shared), B2 = B1 + ns * (nGU + nD);
  // Items below B2 go round-robin (work-group b takes b, b + grid, ...). The routed items, whose cost varies with their
  // group's size, are handed out dynamically: item B2 + x + kDynLists k is the k-th of list x, and the work-groups with
  // blockIdx % kDynLists == x take list x's items in order from its counter (one counter a list keeps the atomics
  // spread; each on a line of its own). A work-group asks for its next item while it runs the current one.
  uint32_t *dyn = p.cnt_dyn + (p.epoch & 1u) * kDynLists * kDynStride;
  if (blockIdx.x == 0 && tid() < kDynLists)
    p.cnt_dyn[(((p.epoch + 1) & 1u) * kDynLists + tid()) * kDynStride] = 0u;
  const uint32_t list = blockIdx.x % kDynLists;
  uint32_t ng = 0xffffffffu, end = 0xffffffffu, grab = 0;
  bool dynamic = false;
  for (uint32_t it = blockIdx.x;;) {
    if (!dynamic && it >= B2) {
      dynamic = true;
      if (tid() == 0) grab = __hip_atomic_fetch_add(dyn + list * kDynStride, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      // The routed groups: every work-group builds the table from the ids once they are all in.
      if (p.route) {
        make_groups(p, lds, &gtab);
        if (blockIdx.x == 0 && tid() == 0) st_co(p.ngroups, gtab.ng);
      } else {
        wait_flag(p, kFlagRouted);
        copy_groups(p, &gtab);
      }
      ng = gtab.ng;
      end = B2 + ng * (nGU + nD) + T * nBlk;
      if (tid() == 0) s_flag = grab;
      __syncthreads();
      it = B2 + list + kDynLists * s_flag;
      __syncthreads();
    }
    if (dynamic) {
      if (it >= end) break;
      if (tid() == 0) grab = __hip_atomic_fetch_add(dyn + list * kDynStride, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    uint64_t *mark = p.trace && it < p.trace_cap ? p.trace + 4 * it : nullptr;
    if (mark && tid() == 0) mark[0] = mark[1] = mark[2] = __builtin_amdgcn_s_memrealtime();
    if (kHc && it < nH) {
      const uint32_t lw = p.hc_lr + kHcStreams;
      if (it < kHcStreams * T)
        hc_norm_item(p, it / kHcStreams, it % kHcStreams, s_part);
      else if (it < kHcStreams * T + lw)
        hc_down_item(p, it - kHcStreams * T, s_part, s_tot, exp_tab, &s_flag);
      else
        hc_up_item(p, it - kHcStreams * T - lw, lds, exp_tab, &s_flag);
    } else if (it < nH + nL) {
      const uint32_t li = it - nH;
      if (kHc) wait_flag(p, kFlagHcX);
      if (p.route) {  // x[li] (its flag tells the shared expert's items), or router row li - T
        if (li < T) {
          quantise_x<kTypes, kHc>(p, li);
          set_flag(p, kFlagLead + li);
        } else {
          const uint32_t r0 = (li - T) * kRouteRows;
          router_rows<kHc>(p, r0, min(kRouteRows, E - r0), (double *)lds);
        }
        if (mark && tid() == 0) mark[2] = __builtin_amdgcn_s_memrealtime();
      } else {
        if (li < T) quantise_x<kTypes, kHc>(p, li);
        if (arrive_last(p.cnt_route, nL, &s_flag)) set_flag(p, kFlagRouted);
      }
    } else if (it < B1) {
      const uint32_t t = it - nH - nL;
      if (kHc) wait_flag(p, kFlagHcX);
      if (mark && tid() == 0) mark[1] = __builtin_amdgcn_s_memrealtime();
      route_token(p, t, exp_tab, s_part, (uint2 *)lds);
      if (mark && tid() == 0) mark[2] = __builtin_amdgcn_s_memrealtime();
      // The shared gate's logit (router row E): gs = sigmoid of it, read only by the combine items. (s_part is
      // route_token's scratch until the barrier.)
      __syncthreads();
      router_dot<kHc>(p, E, t, 1, s_part, s_tot);
      if (tid() == 0) st_tag(p.gs + t, __float_as_uint(sigmoid_libm((float)s_tot[0], exp_tab)), p.tag);
    } else if (it < B2) {
      const uint32_t i = it - B1;
      if (i < ns * nGU) {
        read_group(p, &gtab, true, i / nGU, &sg);
        gate_up_item<kTypes>(p, &sg, i % nGU, lds, grid_lds, &s_grid, exp_tab, mark);
      } else {
        read_group(p, &gtab, true, (i - ns * nGU) / nD, &sg);
        down_item<kTypes>(p, &sg, (i - ns * nGU) % nD, lds, grid_lds, &s_grid, mark);
      }
    } else if (it < B2 + ng * nGU) {
      read_group(p, &gtab, false, (it - B2) / nGU, &sg);
      gate_up_item<kTypes>(p, &sg, (it - B2) % nGU, lds, grid_lds, &s_grid, exp_tab, mark);
    } else {
      const uint32_t i = it - B2 - ng * nGU;
      if (i < ng * nD) {
        read_group(p, &gtab, false, i / nD, &sg);
        down_item<kTypes>(p, &sg, i % nD, lds, grid_lds, &s_grid, mark);
      } else {
        combine_item<kHc>(p, (i - ng * nD) / nBlk, (i - ng * nD) % nBlk, s_wl, exp_tab, mark);
      }
    }
    if (mark && tid() == 0) mark[3] = __builtin_amdgcn_s_memrealtime();
    if (dynamic) {
      if (tid() == 0) s_flag = grab;
      __syncthreads();
      it = B2 + list + kDynLists * s_flag;
    } else {
      it += gridDim.x;
    }
    __syncthreads();
  }
}

// The type sets are instantiated in four translation units that build in parallel: this one (sets 1 - 7, without
// the hyper-connection items, and the dispatch), moe_decode_iq2.hip (sets 8 - 15, the codebook types),
// moe_decode_hc.hip and moe_decode_hc_iq2.hip (sets 1 - 7 and 8 - 15 with them), which include this file.
#define C0VEN_EXTERN(n, hc) extern template __global__ void moe_decode<n, hc>(DecodeParams);
#define C0VEN_INST(n, hc) template __global__ void moe_decode<n, hc>(DecodeParams);
#if defined(C0VEN_DECODE_IQ2_SETS)
#define C0VEN_SET_LO(n) C0VEN_EXTERN(n, false)
#define C0VEN_SET_HI(n) C0VEN_INST(n, false)
#define C0VEN_SET_HC_LO(n) C0VEN_EXTERN(n, true)
#define C0VEN_SET_HC_HI(n) C0VEN_EXTERN(n, true)
#elif defined(C0VEN_DECODE_HC_SETS)
#define C0VEN_SET_LO(n) C0VEN_EXTERN(n, false)
#define C0VEN_SET_HI(n) C0VEN_EXTERN(n, false)
#define C0VEN_SET_HC_LO(n) C0VEN_INST(n, true)
#define C0VEN_SET_HC_HI(n) C0VEN_EXTERN(n, true)
#elif defined(C0VEN_DECODE_HC_IQ2_SETS)
#define C0VEN_SET_LO(n) C0VEN_EXTERN(n, false)
#define C0VEN_SET_HI(n) C0VEN_EXTERN(n, false)
#define C0VEN_SET_HC_LO(n) C0VEN_EXTERN(n, true)
#define C0VEN_SET_HC_HI(n) C0VEN_INST(n, true)
#else
#define C0VEN_SET_LO(n) C0VEN_INST(n, false)
#define C0VEN_SET_HI(n) C0VEN_EXTERN(n, false)
#define C0VEN_SET_HC_LO(n) C0VEN_EXTERN(n, true)
#define C0VEN_SET_HC_HI(n) C0VEN_EXTERN(n, true)
#endif
C0VEN_SET_LO(1)
C0VEN_SET_LO(2)
C0VEN_SET_LO(3)
C0VEN_SET_LO(4)
C0VEN_SET_LO(5)
C0VEN_SET_LO(6)
C0VEN_SET_LO(7)
C0VEN_SET_HI(8)
C0VEN_SET_HI(9)
C0VEN_SET_HI(10)
C0VEN_SET_HI(11)
C0VEN_SET_HI(12)
C0VEN_SET_HI(13)
C0VEN_SET_HI(14)
C0VEN_SET_HI(15)
C0VEN_SET_HC_LO(1)
C0VEN_SET_HC_LO(2)
C0VEN_SET_HC_LO(3)
C0VEN_SET_HC_LO(4)
C0VEN_SET_HC_LO(5)
C0VEN_SET_HC_LO(6)
C0VEN_SET_HC_LO(7)
C0VEN_SET_HC_HI(8)
C0VEN_SET_HC_HI(9)
C0VEN_SET_HC_HI(10)
C0VEN_SET_HC_HI(11)
C0VEN_SET_HC_HI(12)
C0VEN_SET_HC_HI(13)
C0VEN_SET_HC_HI(14)
C0VEN_SET_HC_HI(15)
#undef C0VEN_SET_LO
#undef C0VEN_SET_HI
#undef C0VEN_SET_HC_LO
#undef C0VEN_SET_HC_HI
#undef C0VEN_EXTERN
#undef C0VEN_INST

#if !defined(C0VEN_DECODE_IQ2_SETS) && !defined(C0VEN_DECODE_HC_SETS) && !defined(C0VEN_DECODE_HC_IQ2_SETS)
const void *decode_kernel(uint32_t types, bool hc) {
  switch (types + (hc ? 16 : 0)) {
    case 1: return (const void *)moe_decode<1, false>;
    case 2: return (const void *)moe_decode<2, false>;
    case 3: return (const void *)moe_decode<3, false>;
    case 4: return (const void *)moe_decode<4, false>;
    case 5: return (const void *)moe_decode<5, false>;
    case 6: return (const void *)moe_decode<6, false>;
    case 7: return (const void *)moe_decode<7, false>;
    case 8: return (const void *)moe_decode<8, false>;
    case 9: return (const void *)moe_decode<9, false>;
    case 10: return (const void *)moe_decode<10, false>;
    case 11: return (const void *)moe_decode<11, false>;
    case 12: return (const void *)moe_decode<12, false>;
    case 13: return (const void *)moe_decode<13, false>;
    case 14: return (const void *)moe_decode<14, false>;
    case 15: return (const void *)moe_decode<15, false>;
    case 17: return (const void *)moe_decode<1, true>;
    case 18: return (const void *)moe_decode<2, true>;
    case 19: return (const void *)moe_decode<3, true>;
    case 20: return (const void *)moe_decode<4, true>;
    case 21: return (const void *)moe_decode<5, true>;
    case 22: return (const void *)moe_decode<6, true>;
    case 23: return (const void *)moe_decode<7, true>;
    case 24: return (const void *)moe_decode<8, true>;
    case 25: return (const void *)moe_decode<9, true>;
    case 26: return (const void *)moe_decode<10, true>;
    case 27: return (const void *)moe_decode<11, true>;
    case 28: return (const void *)moe_decode<12, true>;
    case 29: return (const void *)moe_decode<13, true>;
    case 30: return (const void *)moe_decode<14, true>;
    case 31: return (const void *)moe_decode<15, true>;
    default: return nullptr;
  }
}
#endif

}  // namespace c0ven
