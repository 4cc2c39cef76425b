// The decode-shape MoE block (a few tokens: decode and speculative verify) as one persistent kernel.
//
// Replaces the reference's decode kernel list for the block (model.cpp:1348-1414): the router's bf16 GEMV
// (mv_xmx_bf16), router_group (layer.cl:984-1023), moe_gate_up_g (moe.cl:230-302), moe_down_g (moe.cl:416-471) and
// moe_combine (layer.cl:869-884). Every work-group walks the work items b, b + grid, b + 2 grid, ... in one order
// (decode.h): lead items (router rows; x quantised), top-k items, gate/up items, down items. An item that needs earlier
// work waits on flags set (to this launch's epoch) by the work it needs:
//   - each lead item sets its own flag; a top-k item waits for all of them (no counter the lead items contend on);
//   - the last top-k item in groups the assignments into MoeGroups and sets "routed" (gate/up items wait on it);
//   - the last gate/up item of a 256-row unit of group g quantises that unit of h for the down; the last unit sets
//     group g's flag (its down items wait on it);
//   - the last down item of a (token, row block) to finish combines that token's rows: sum_k w_k y_k + gs s.
// Every item's dependencies have smaller indices, and a work-group takes its items in increasing order, so the
// smallest unfinished item always has everything it waits for once every work-group runs: the grid is no larger than
// what the device holds at once, so each is dispatched (behind other streams' kernels at worst, which do not wait on
// this one). A cooperative launch would state the same guarantee but costs ~20 us more per launch on this runtime.
// Waits are bounded anyway: past kSpinLimit polls a wait gives up and sets *err.
#include <hip/hip_runtime.h>

#include "act_quant.h"
#include "decode.h"
#include "route.h"
#include "device_math.h"
#include "iq3s_grid.h"
#include "layout.h"
#include "units.h"

namespace c0ven {

__device__ __constant__ static const uint32_t kIq3sGridDev[512] = {C0VEN_IQ3S_GRID_VALUES};

namespace {

constexpr uint32_t kSpinLimit = 1u << 22;
#ifndef C0VEN_POLL_SLEEP
#define C0VEN_POLL_SLEEP 1
#endif

__device__ __forceinline__ uint32_t lane_id() { return threadIdx.x & 63u; }
__device__ __forceinline__ uint32_t wave_id() { return threadIdx.x >> 6; }

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
  if (threadIdx.x == 0) {
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
  if (threadIdx.x == 0) st_co(p.flags + i, p.epoch);
}

// Waits until flag i holds this launch's epoch (thread 0 polls, the work-group follows).
__device__ __forceinline__ void wait_flag(const DecodeParams &p, uint32_t i) {
  if (threadIdx.x == 0) {
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

// Waits until flags base .. base + count - 1 (count <= kMaxLeadItems) all hold this launch's epoch (wave 0 polls,
// a flag a lane, all loads of a round in flight together; the work-group follows).
__device__ __forceinline__ void wait_flags(const DecodeParams &p, uint32_t base, uint32_t count) {
  if (wave_id() == 0) {
    uint32_t n = 0;
    for (;;) {
      bool ok = true;
#pragma unroll
      for (uint32_t i = 0; i < (kMaxLeadItems + 63) / 64; i++) {
        const uint32_t f = lane_id() + 64 * i;
        if (f < count) ok &= ld_co(p.flags + base + f) == p.epoch;
      }
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

// Top-k and weights for token t (route.h:39-99 and layer.cl:765-804 restated). Two waves at once: wave 1 takes the
// softmax's max and 1 / sum (the sum in double); wave 0 selects: lane l holds
// experts l + 64 i, sorted by (logit, lower id first), and each of the k rounds takes the wave's largest head (a DPP
// max of the logit keys, a ballot for equal keys, the lower id among them) and pops it. Then wave 0 turns the k
// winners into weights. The winners' ids and keys stay in sel (sel[j], sel[kMaxUsed + j]) for the grouping.
__device__ __forceinline__ void route_token(const DecodeParams &p, uint32_t t, const uint64_t *tab, uint32_t *sel, float *norm) {
  const uint32_t lane = lane_id(), E = p.E, K = p.K;
  const float *lg = p.logits + (uint64_t)t * (E + 1);
  uint32_t my_id = 0, my_key = 0;
  if (wave_id() <= 1) {
    uint32_t key[kRoutePer], id[kRoutePer];
    route_load(lg, E, lane, key, id);
    if (wave_id() == 1) {
      float mx, inv;
      route_norm(key, E, lane, tab, &mx, &inv);
      if (lane == 0) norm[0] = mx, norm[1] = inv;
    } else {
      route_select(key, id, K, lane, &my_id, &my_key);
      if (lane < K) sel[lane] = my_id, sel[kMaxUsed + lane] = my_key;
    }
  }
  __syncthreads();
  if (wave_id() == 0) {
    const float w = route_weight(my_key, norm[0], norm[1], K, lane, tab);
    if (lane < K) {
      st_co(p.ids + t * K + lane, (int32_t)my_id);
      st_co(p.w + t * K + lane, w);
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
    m.type = which == 2 ? p.sh_down_type : p.sh_gate_type;
    m.mat = p.shared + (which == 0 ? 0 : which == 1 ? p.sh_up_off : p.sh_down_off);
  } else {
    m.type = which == 2 ? p.down_type : p.gate_type;
    m.mat = p.experts + (uint64_t)slot * p.ex_bytes + (which == 0 ? 0 : which == 1 ? p.ex_up_off : p.ex_down_off);
  }
  return m;
}

__device__ __forceinline__ uint32_t asg_token(const DecodeParams &p, uint32_t asg) {
  const uint32_t n = p.T * p.K;
  return asg < n ? asg / p.K : asg - n;
}

__device__ __forceinline__ void load_grid(uint32_t *grid_lds) {
  for (uint32_t i = threadIdx.x; i < 512; i += kWG) grid_lds[i] = kIq3sGridDev[i];
}

// The n terms of one (row, unit) pair against the activation units act + j * stride dwords, into t[j]. The unit's
// weights are loaded first; `ready` (run by the whole work-group) then makes the activations available, so the
// weights' HBM latency overlaps whatever ready waits for.
template <uint32_t kTypes, typename Ready>
__device__ __forceinline__ void pair_terms(uint32_t type, const uint8_t *tile, uint32_t idx, uint32_t nl,
                                           const uint32_t *grid_lds, const uint32_t *act, uint32_t stride,
                                           const uint32_t &n, float *t, Ready ready) {
  if constexpr ((kTypes & kTypeQ8_0) != 0) {
    if (kTypes == kTypeQ8_0 || type == QT_Q8_0) {
      UnitQ8_0 w;
      w.load(tile, idx, nl);
      ready();
#pragma unroll
      for (uint32_t j = 0; j < MOE_GROUP_MAX; j++)
        if (j < n) t[j] = w.term(Act(act + j * stride));
      return;
    }
  }
  if constexpr ((kTypes & kTypeQ4_K) != 0) {
    if ((kTypes & ~kTypeQ8_0) == kTypeQ4_K || type == QT_Q4_K) {
      UnitQ4_K w;
      w.load(tile, idx, nl);
      ready();
#pragma unroll
      for (uint32_t j = 0; j < MOE_GROUP_MAX; j++)
        if (j < n) t[j] = w.term(Act(act + j * stride));
      return;
    }
  }
  if constexpr ((kTypes & kTypeIQ3_S) != 0) {
    UnitIQ3_S w;
    w.load(tile, idx, nl, grid_lds);
    ready();
#pragma unroll
    for (uint32_t j = 0; j < MOE_GROUP_MAX; j++)
      if (j < n) t[j] = w.term(Act(act + j * stride));
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
template <uint32_t kTypes>
__device__ __forceinline__ void quantise_x(const DecodeParams &p, uint32_t t) {
  const uint32_t H = p.H, l32 = threadIdx.x & 31u;
  for (uint32_t u = threadIdx.x / 32; u < H / kUnit; u += kWG / 32) {
    const float4 *src = (const float4 *)(p.x + (uint64_t)t * H + u * kUnit + 8 * l32);
    const float4 a = src[0], b = src[1];
    const float v[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
    quant_unit(v, l32, act_type<kTypes>(p.xact_r), p.act_r + ((uint64_t)t * (H / kUnit) + u) * kActBytes);
    if (p.act_s != p.act_r) quant_unit(v, l32, act_type<kTypes>(p.xact_s), p.act_s + ((uint64_t)t * (H / kUnit) + u) * kActBytes);
  }
}

// Router row dot products with tokens t_begin .. t_end - 1, in part[wave][t]: wave w takes row `row`'s 512-value
// chunks c0, c0 + step, ..., a lane eight values of each, every product bf16(W) bf16(x) exact and summed in fp64 (the lane's share,
// then the wave's in a fixed order). x is read straight from global memory (it is L2-resident: every lead item reads
// it), four tokens' worth in flight at once.
__device__ __forceinline__ void row_dots(const DecodeParams &p, uint32_t row, uint32_t c0, uint32_t step,
                                         uint32_t t_begin, uint32_t t_end, double *part) {
  const uint32_t lane = lane_id(), wv = wave_id(), H = p.H, nC = H / 512;
  const uint16_t *wr = p.router + (uint64_t)row * H + lane * 8;
  const float *xl = p.x + lane * 8;
  const uint32_t c1 = c0 + step;  // the wave's first two chunks stay in registers, their x loads in flight together
  const uint4 w0 = c0 < nC ? *(const uint4 *)(wr + 512 * c0) : make_uint4(0, 0, 0, 0);
  const uint4 w1 = c1 < nC ? *(const uint4 *)(wr + 512 * c1) : make_uint4(0, 0, 0, 0);
  auto fma8 = [](const uint4 &wq, const float4 &xa, const float4 &xb, double acc) {
    const uint32_t ww[4] = {wq.x, wq.y, wq.z, wq.w};
    const float xs[8] = {xa.x, xa.y, xa.z, xa.w, xb.x, xb.y, xb.z, xb.w};
#pragma unroll
    for (int k = 0; k < 8; k++) {
      const double wd = (double)__uint_as_float((k & 1) ? ww[k / 2] & 0xffff0000u : ww[k / 2] << 16);
      acc = __builtin_fma(wd, (double)round_bf16(xs[k]), acc);
    }
    return acc;
  };
  for (uint32_t t0 = t_begin; t0 < t_end; t0 += 4) {
    float4 xa[4], xb[4], ya[4], yb[4];
#pragma unroll
    for (uint32_t tt = 0; tt < 4; tt++) {
      const float *xt = xl + (uint64_t)min(t0 + tt, t_end - 1) * H;
      const float4 *q = (const float4 *)(xt + 512 * min(c0, nC - 1));
      const float4 *q1 = (const float4 *)(xt + 512 * min(c1, nC - 1));
      xa[tt] = q[0], xb[tt] = q[1], ya[tt] = q1[0], yb[tt] = q1[1];
    }
    double acc[4] = {0.0, 0.0, 0.0, 0.0};
    if (c0 < nC) {
#pragma unroll
      for (uint32_t tt = 0; tt < 4; tt++) acc[tt] = fma8(w0, xa[tt], xb[tt], acc[tt]);
    }
    if (c1 < nC) {
#pragma unroll
      for (uint32_t tt = 0; tt < 4; tt++) acc[tt] = fma8(w1, ya[tt], yb[tt], acc[tt]);
    }
    for (uint32_t c = c1 + step; c < nC; c += step) {  // long rows
      const uint4 wq = *(const uint4 *)(wr + 512 * c);
#pragma unroll
      for (uint32_t tt = 0; tt < 4; tt++) {
        const float4 *q = (const float4 *)(xl + (uint64_t)min(t0 + tt, t_end - 1) * H + 512 * c);
        acc[tt] = fma8(wq, q[0], q[1], acc[tt]);
      }
    }
#pragma unroll
    for (uint32_t tt = 0; tt < 4; tt++) {
      const double sum = wave_sum_f64(acc[tt]);
      if (lane == 0 && t0 + tt < t_end) part[wv * kMaxDecodeTokens + t0 + tt] = sum;
    }
  }
  __syncthreads();
}

// The four waves' sums of token t, in a fixed order (the shared gate's row).
__device__ __forceinline__ float row_total4(const double *part, uint32_t t) {
  return (float)__dadd_rn(__dadd_rn(part[t], part[kMaxDecodeTokens + t]),
                          __dadd_rn(part[2 * kMaxDecodeTokens + t], part[3 * kMaxDecodeTokens + t]));
}

// Lead item i: router rows 2 i and 2 i + 1 (waves 2 r and 2 r + 1 take the even and odd chunks of row 2 i + r) for all
// T tokens, plus the bias.
__device__ __forceinline__ void router_rows(const DecodeParams &p, uint32_t item, double *part) {
  const uint32_t r = wave_id() / 2, row = min(item * kRouteRows + r, p.E - 1);
  row_dots(p, row, wave_id() & 1u, 2, 0, p.T, part);
  const uint32_t j = threadIdx.x, rr = j / p.T, t = j % p.T, rw = item * kRouteRows + rr;
  if (j < kRouteRows * p.T && rw < p.E) {
    float l = (float)__dadd_rn(part[2 * rr * kMaxDecodeTokens + t], part[(2 * rr + 1) * kMaxDecodeTokens + t]);
    if (p.bias) l = __fadd_rn(l, p.bias[rw]);
    st_co(p.logits + (uint64_t)t * (p.E + 1) + rw, l);
  }
}

// MoeGroup records from the routed ids: an expert's assignments in order, MOE_GROUP_MAX a group (as group_slots,
// layer.cl:894-942), and the shared expert's groups; numbered by decreasing size, then by first assignment. An expert takes at
// most one assignment a token, so a mask of the tokens that chose it gives each assignment its rank among the
// expert's (and whether it heads a group); the heads' ballots give the group numbers. Token own's ids come from sel,
// the others' from the coherent ids.
__device__ __forceinline__ void make_groups(const DecodeParams &p, uint32_t own, const uint32_t *sel, uint8_t *lds, uint64_t *hb) {
  const uint32_t T = p.T, K = p.K, E = p.E, n = T * K, a = threadIdx.x, lane = lane_id();
  uint32_t *ids = (uint32_t *)lds, *mask = ids + kMaxDecodeTokens * kMaxUsed, *gnum = mask + kMaxExperts;
  for (uint32_t i = a; i < E; i += kWG) mask[i] = 0u;
  const uint32_t t = a / K;
  if (a < n) ids[a] = t == own ? sel[a % K] : (uint32_t)ld_co(p.ids + a);
  __syncthreads();
  uint32_t e = 0, rank = 0, total = 0;
  if (a < n) {
    e = ids[a];
    atomicOr(mask + e, 1u << t);
  }
  __syncthreads();
  if (a < n) {
    const uint32_t m = mask[e];
    rank = __popc(m & ((1u << t) - 1u));
    total = __popc(m);
  }
  const bool head = a < n && rank % MOE_GROUP_MAX == 0;
  const uint64_t heads = __ballot(head);
  if (lane == 0) hb[wave_id()] = heads;
  __syncthreads();
  uint32_t before = 0, nr = 0;
#pragma unroll
  for (uint32_t w = 0; w < kWG / 64; w++) {
    const uint32_t c = (uint32_t)__popcll(hb[w]);
    before += w < wave_id() ? c : 0u;
    nr += c;
  }
  // Groups in order of first assignment (routed, then the shared expert's) get the index o; they are numbered by
  // decreasing size, o breaking ties, so that the heaviest groups' items come first (work-groups take items in index
  // order).
  const uint32_t ns = p.has_shared ? (T + MOE_GROUP_MAX - 1) / MOE_GROUP_MAX : 0, G = nr + ns;
  uint32_t *gkey = gnum + 2 * kMaxExperts;
  uint32_t o = 0, gn = 0;
  if (head) {
    o = before + __builtin_amdgcn_mbcnt_hi((uint32_t)(heads >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)heads, 0u));
    gn = min((uint32_t)MOE_GROUP_MAX, total - rank);
    gkey[o] = (MOE_GROUP_MAX - gn) * 1024u + o;
  }
  const uint32_t sn = a < ns ? min((uint32_t)MOE_GROUP_MAX, T - a * MOE_GROUP_MAX) : 0u;
  if (a < ns) gkey[nr + a] = (MOE_GROUP_MAX - sn) * 1024u + nr + a;
  __syncthreads();
  auto order = [&](uint32_t key) {
    uint32_t r = 0;
    for (uint32_t i = 0; i < G; i++) r += gkey[i] < key;
    return r;
  };
  if (head) {
    const uint32_t g = order((MOE_GROUP_MAX - gn) * 1024u + o);
    gnum[2 * e + rank / MOE_GROUP_MAX] = g;
    st_co(&p.groups[g].slot, (int32_t)e);
    st_co(&p.groups[g].n, gn);
  }
  if (a < ns) {
    MoeGroup *g = p.groups + order((MOE_GROUP_MAX - sn) * 1024u + nr + a);
    st_co(&g->slot, (int32_t)E);
    st_co(&g->n, sn);
    for (uint32_t j = 0; j < MOE_GROUP_MAX; j++)
      if (a * MOE_GROUP_MAX + j < T) st_co(g->asg + j, n + a * MOE_GROUP_MAX + j);
  }
  __syncthreads();
  if (a < n) st_co(p.groups[gnum[2 * e + rank / MOE_GROUP_MAX]].asg + rank % MOE_GROUP_MAX, a);
  if (a == 0) st_co(p.ngroups, nr + ns);
}

// ---------------------------------------------------------------------------------------------------------------
// Expert items

struct GroupLds {
  int32_t slot;
  uint32_t n, asg[MOE_GROUP_MAX], tok[MOE_GROUP_MAX];
};

__device__ __forceinline__ void read_group(const DecodeParams &p, uint32_t g, GroupLds *s) {
  const MoeGroup *grp = p.groups + g;
  if (threadIdx.x == 0) s->slot = ld_co(&grp->slot), s->n = ld_co(&grp->n);
  if (threadIdx.x < MOE_GROUP_MAX) {
    const uint32_t a = ld_co(grp->asg + threadIdx.x);
    s->asg[threadIdx.x] = a;
    s->tok[threadIdx.x] = asg_token(p, a);
  }
  __syncthreads();
}

// Activation units (act + unit index * kActBytes, coherent) of the group's assignments into LDS, kActLds apart.
__device__ __forceinline__ void stage_act(const uint8_t *act, const uint32_t *unit_of_j, uint32_t n, uint32_t U,
                                          uint8_t *lds) {
  for (uint32_t i = threadIdx.x; i < n * U * (kActBytes / 16); i += kWG) {
    const uint32_t unit = i / (kActBytes / 16), c = i % (kActBytes / 16), j = unit / U, u = unit % U;
    *(uint4 *)(lds + unit * kActLds + 16 * c) = ld_co4(act + ((uint64_t)unit_of_j[j] * U + u) * kActBytes + 16 * c);
  }
}

// Gate and up of rows blk * gate_up_rows .. of group g: lane = m * 32 + r * U + u; h = silu(g) * u per row.
template <uint32_t kTypes>
__device__ __forceinline__ void gate_up_item(const DecodeParams &p, uint32_t g, uint32_t blk, uint8_t *lds, uint32_t *grid_lds,
                             GroupLds *sg, uint32_t *s_flag, const uint64_t *tab, uint64_t *mark) {
  read_group(p, g, sg);
  const uint32_t U = p.H / kUnit, rows = gate_up_rows(U), row0 = blk * rows, n = sg->n;
  const GroupMat gm = group_mat(p, sg->slot, 0);
  if ((kTypes & kTypeIQ3_S) && gm.type == QT_IQ3_S) {
    load_grid(grid_lds);
    __syncthreads();
  }
  const uint32_t lane = lane_id(), m = lane / 32, r = (lane % 32) / U, u = lane % U;
  const uint32_t row = row0 + wave_id() * (32 / U) + r;
  const uint8_t *mat = gm.mat + (m ? (gm.shared ? p.sh_up_off : p.ex_up_off) : 0);
  const uint8_t *tile = mat + (uint64_t)(row / kTileRows) * tile_bytes(gm.type, U);
  float t[MOE_GROUP_MAX];
  pair_terms<kTypes>(gm.type, tile, (row % kTileRows) * U + u, kTileRows * U, grid_lds,
             (const uint32_t *)lds + u * (kActLds / 4), U * (kActLds / 4), n, t, [&] {
               stage_act(gm.shared ? p.act_s : p.act_r, sg->tok, n, U, lds);
               __syncthreads();
               if (mark && threadIdx.x == 0) mark[1] = __builtin_amdgcn_s_memrealtime();
             });
#pragma unroll
  for (uint32_t j = 0; j < MOE_GROUP_MAX; j++) {
    if (j >= n) break;
    const float s = row_sum(t[j], U);        // gate's row sum in lanes m = 0, up's in m = 1
    const float su = __shfl_xor(s, 32, 64);  // the other matrix's
    if (m == 0 && u == 0) st_co(p.h + (uint64_t)sg->asg[j] * p.F + row, swiglu_one(s, su, p.swiglu_limit, tab));
  }
  if (mark && threadIdx.x == 0) mark[2] = __builtin_amdgcn_s_memrealtime();
  // The last item of these 256 rows quantises them, one unit of the down's K per assignment, a half-wave each; the
  // last unit of the group sets its flag.
  const uint32_t Ud = p.F / kUnit, unit = row0 / kUnit;
  if (!arrive_last(p.cnt_hu + (uint64_t)g * Ud + unit, kUnit / rows, s_flag)) return;
  const uint32_t j = threadIdx.x / 32, l32 = threadIdx.x & 31u;
  if (j < n) {
    const float *src = p.h + (uint64_t)sg->asg[j] * p.F + unit * kUnit + 8 * l32;
    float v[8];
#pragma unroll
    for (int i = 0; i < 8; i++) v[i] = ld_co(src + i);
    const uint32_t dact = act_type<kTypes>(quant_vec_dot_type(group_mat(p, sg->slot, 2).type));
    quant_unit(v, l32, dact, p.hact + ((uint64_t)sg->asg[j] * Ud + unit) * kActBytes);
  }
  if (arrive_last(p.cnt_hq + g, Ud, s_flag)) set_flag(p, kFlagH + g);
}

// Down rows blk * down_rows .. of group g (lane = r * U + u), then the combine of every token this item completes.
template <uint32_t kTypes>
__device__ __forceinline__ void down_item(const DecodeParams &p, uint32_t g, uint32_t blk, uint8_t *lds, uint32_t *grid_lds,
                          GroupLds *sg, uint32_t *s_last, uint64_t *mark) {
  read_group(p, g, sg);
  const uint32_t U = p.F / kUnit, rows = down_rows(U), row0 = blk * rows, n = sg->n, nblk = p.H / rows;
  const GroupMat gm = group_mat(p, sg->slot, 2);
  if ((kTypes & kTypeIQ3_S) && gm.type == QT_IQ3_S) {
    load_grid(grid_lds);
    __syncthreads();
  }
  const uint32_t lane = lane_id(), r = lane / U, u = lane % U;
  const uint32_t row = row0 + wave_id() * (64 / U) + r;
  const uint8_t *tile = gm.mat + (uint64_t)(row / kTileRows) * tile_bytes(gm.type, U);
  float t[MOE_GROUP_MAX];
  pair_terms<kTypes>(gm.type, tile, (row % kTileRows) * U + u, kTileRows * U, grid_lds,
             (const uint32_t *)lds + u * (kActLds / 4), U * (kActLds / 4), n, t, [&] {
               wait_flag(p, kFlagH + g);  // the weights are already on their way
               stage_act(p.hact, sg->asg, n, U, lds);
               __syncthreads();
               if (mark && threadIdx.x == 0) mark[1] = __builtin_amdgcn_s_memrealtime();
             });
#pragma unroll
  for (uint32_t j = 0; j < MOE_GROUP_MAX; j++) {
    if (j >= n) break;
    const float s = row_sum(t[j], U);
    if (u == 0) st_co(p.y_asg + (uint64_t)sg->asg[j] * p.H + row, s);
  }
  if (mark && threadIdx.x == 0) mark[2] = __builtin_amdgcn_s_memrealtime();
  // Count this item's outputs in, one counter per (token, row block), all at once.
  stores_done();
  if (threadIdx.x < n) {
    const uint32_t tk = sg->tok[threadIdx.x];
    const uint32_t need = p.tok_need ? p.tok_need[tk] : p.K + (p.has_shared ? 1u : 0u);
    uint32_t *cnt = p.cnt_tok + (uint64_t)tk * nblk + blk;
    const uint32_t old = __hip_atomic_fetch_add(cnt, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    s_last[threadIdx.x] = old == need - 1;
    if (old == need - 1) __hip_atomic_store(cnt, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  __syncthreads();
  // The completed tokens' rows, a (token, row) pair a thread: y = sum_k w_k y_k in rank order, then + gs s; every
  // operand loaded first, then summed in order.
  uint32_t done[MOE_GROUP_MAX], nd = 0;
  for (uint32_t j = 0; j < n; j++)
    if (s_last[j]) done[nd++] = sg->tok[j];
  for (uint32_t i = threadIdx.x; i < nd * rows; i += kWG) {
    const uint32_t tk = done[i / rows], rr = row0 + i % rows, K = p.K;
    float yv[kMaxUsed], wv[kMaxUsed];
    bool on[kMaxUsed];
#pragma unroll
    for (uint32_t k = 0; k < kMaxUsed; k++) {
      on[k] = k < K && (p.route || ld_co(p.ids + tk * K + k) >= 0);
      wv[k] = k < K ? ld_co(p.w + tk * K + k) : 0.0f;
      yv[k] = on[k] ? ld_co(p.y_asg + ((uint64_t)tk * K + k) * p.H + rr) : 0.0f;
    }
    const float ys = p.has_shared ? ld_co(p.y_asg + ((uint64_t)p.T * K + tk) * p.H + rr) : 0.0f;
    const float gs = p.has_shared ? ld_co(p.gs + tk) : 0.0f;
    float acc = 0.0f;
#pragma unroll
    for (uint32_t k = 0; k < kMaxUsed; k++)
      if (on[k]) acc = __fadd_rn(acc, __fmul_rn(wv[k], yv[k]));
    if (p.has_shared) acc = __fadd_rn(acc, __fmul_rn(gs, ys));
    p.y[(uint64_t)tk * p.H + rr] = acc;
  }
}

}  // namespace

// Grid: the work-groups of 256 the device holds at once; dynamic LDS: the larger of a group's activation units
// (MOE_GROUP_MAX x units x kActLds) and the grouping's tables (kGroupingLds).
template <uint32_t kTypes>
__global__ void __launch_bounds__(kWG) __attribute__((amdgpu_waves_per_eu(2))) moe_decode(DecodeParams p) {
  extern __shared__ __align__(16) uint8_t lds[];
  __shared__ uint32_t grid_lds[512];
  __shared__ uint32_t s_flag, s_ng, s_last[MOE_GROUP_MAX], s_sel[2 * kMaxUsed];
  __shared__ float s_norm[2];
  __shared__ uint64_t s_hb[kWG / 64];
  __shared__ double s_part[(kWG / 64) * kMaxDecodeTokens];
  __shared__ GroupLds sg;
  __shared__ uint64_t exp_tab[32];  // expf's table, read at LDS latency
  if (threadIdx.x < 32) exp_tab[threadIdx.x] = kExp2Tab[threadIdx.x];
  __syncthreads();
  const uint32_t T = p.T, E = p.E, Ug = p.H / kUnit, Ud = p.F / kUnit;
  const uint32_t nL = lead_items(T, E, p.route), nTop = p.route ? T : 0, B1 = nL + nTop;
  const uint32_t nGU = p.F / gate_up_rows(Ug), nD = p.H / down_rows(Ud);
  uint32_t ng = 0xffffffffu, end = 0xffffffffu;
  for (uint32_t it = blockIdx.x;; it += gridDim.x) {
    if (it >= B1) {
      if (ng == 0xffffffffu) {
        wait_flag(p, kFlagRouted);
        if (threadIdx.x == 0) s_ng = ld_co(p.ngroups);
        __syncthreads();
        ng = s_ng;
        end = B1 + ng * (nGU + nD);
      }
      if (it >= end) break;
    }
    uint64_t *mark = p.trace && it < p.trace_cap ? p.trace + 4 * it : nullptr;
    if (mark && threadIdx.x == 0) mark[0] = mark[1] = mark[2] = __builtin_amdgcn_s_memrealtime();
    if (it < nL) {
      if (it < T) quantise_x<kTypes>(p, it);
      if (p.route) {
        if (it * kRouteRows < E) router_rows(p, it, s_part);
        if (mark && threadIdx.x == 0) mark[2] = __builtin_amdgcn_s_memrealtime();
        set_flag(p, kFlagLead + it);
      } else if (arrive_last(p.cnt_route, nL, &s_flag)) {
        set_flag(p, kFlagRouted);
      }
    } else if (it < B1) {
      const uint32_t t = it - nL;
      // The shared gate's logit (router row E) for this token while the lead items finish: gs = sigmoid of it.
      row_dots(p, E, wave_id(), 4, t, t + 1, s_part);
      if (threadIdx.x == 0) st_co(p.gs + t, sigmoid_libm(row_total4(s_part, t), exp_tab));
      wait_flags(p, kFlagLead, nL);
      if (mark && threadIdx.x == 0) mark[1] = __builtin_amdgcn_s_memrealtime();
      route_token(p, t, exp_tab, s_sel, s_norm);
      if (mark && threadIdx.x == 0) mark[2] = __builtin_amdgcn_s_memrealtime();
      if (T == 1 || arrive_last(p.cnt_topk, T, &s_flag)) {
        make_groups(p, t, s_sel, lds, s_hb);
        set_flag(p, kFlagRouted);
      }
    } else if (it < B1 + ng * nGU) {
      gate_up_item<kTypes>(p, (it - B1) / nGU, (it - B1) % nGU, lds, grid_lds, &sg, &s_flag, exp_tab, mark);
    } else {
      const uint32_t i = it - B1 - ng * nGU;
      down_item<kTypes>(p, i / nD, i % nD, lds, grid_lds, &sg, s_last, mark);
    }
    if (mark && threadIdx.x == 0) mark[3] = __builtin_amdgcn_s_memrealtime();
    __syncthreads();
  }
}

template __global__ void moe_decode<1>(DecodeParams);
template __global__ void moe_decode<2>(DecodeParams);
template __global__ void moe_decode<3>(DecodeParams);
template __global__ void moe_decode<4>(DecodeParams);
template __global__ void moe_decode<5>(DecodeParams);
template __global__ void moe_decode<6>(DecodeParams);
template __global__ void moe_decode<7>(DecodeParams);

const void *decode_kernel(uint32_t types) {
  switch (types) {
    case 1: return (const void *)moe_decode<1>;
    case 2: return (const void *)moe_decode<2>;
    case 3: return (const void *)moe_decode<3>;
    case 4: return (const void *)moe_decode<4>;
    case 5: return (const void *)moe_decode<5>;
    case 6: return (const void *)moe_decode<6>;
    default: return (const void *)moe_decode<7>;
  }
}

}  // namespace c0ven
