// The decode-shape MoE block (a few tokens: decode and speculative verify) as three launches on one stream:
//
//   moe_route      the router's bf16 GEMV (fp64 accumulation), the activations quantised, and in the last work-group
//                  to finish: softmax, top-k, weights and the MoeGroup records (replaces router_group, layer.cl:984-1023,
//                  and the router's mv_xmx_bf16, model.cpp:1354);
//   moe_gate_up    gate and up of every group's expert (a wave per 64-row x 256-value tile, the weights decoded once for
//                  the group's assignments), and in the last work-group of each 256 rows: the pairwise sum over units,
//                  SwiGLU and h quantised to the down's activation type (replaces moe_gate_up_g, moe.cl:230-302);
//   moe_down       down for every group, and in the last work-group of each 256 rows: the sum over units, then for a
//                  token whose k + 1 outputs are all done, the combine sum_k w_k y_k + gs s in rank order (replaces
//                  moe_down_g, moe.cl:416-471, and moe_combine, layer.cl:869-884).
//
// "Last work-group" is an arrival counter per piece of work: each work-group writes its share, fences at device scope
// and counts itself in; the one that brings the count to the total does the finishing step and sets the counter back
// to zero for the next launch. Nothing waits on another work-group, so no launch depends on residency.
#include <hip/hip_runtime.h>

#include "decode.h"
#include "device_math.h"
#include "iq3s_grid.h"
#include "layout.h"
#include "units.h"

namespace c0ven {

__device__ __constant__ static const uint32_t kIq3sGridDev[512] = {C0VEN_IQ3S_GRID_VALUES};

namespace {

constexpr uint32_t kRouteWG = 512;  // threads of the router's work-groups: eight waves

__device__ __forceinline__ uint32_t lane_id() { return threadIdx.x & 63u; }
__device__ __forceinline__ uint32_t wave_id() { return threadIdx.x >> 6; }

// Data one work-group writes and another reads within a launch goes through device-coherent accesses (agent-scope
// relaxed atomics: the store writes through the XCD's L2, the load reads past a stale line), so no fence has to
// write back or invalidate a whole L2.
__device__ __forceinline__ void st_co(float *p, float v) { __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }
__device__ __forceinline__ float ld_co(const float *p) {
  return __hip_atomic_load(const_cast<float *>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Counts the work-group in on *cnt once its coherent stores have completed; true in every thread of the one that
// completes `total` (which sets the counter back to zero).
__device__ __forceinline__ bool arrive_last(uint32_t *cnt, uint32_t total, uint32_t *flag) {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
  __builtin_amdgcn_s_waitcnt(0);  // this wave's stores are done
  __syncthreads();
  if (threadIdx.x == 0) {
    const uint32_t old = __hip_atomic_fetch_add(cnt, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    *flag = old == total - 1;
    if (old == total - 1) __hip_atomic_store(cnt, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  __syncthreads();
  return *flag != 0;
}

// One activation unit (256 values) quantised by a half-wave, eight values a lane (lane l32 holds values 8 l32..+7),
// with the CPU path's rules: q8_K (quantize_row_q8_K_ref) or q8_0 (the x86 quantize_row_q8_0).
__device__ void quant_unit(const float v[8], uint32_t l32, uint32_t act_type, uint8_t *out) {
  uint32_t code[2] = {0u, 0u};
  if (act_type == QT_Q8_K) {
    // The value of largest magnitude, the first of equals: (|v|, index) reduced over the 32 lanes.
    float amax = 0.0f, mx = 0.0f;
    uint32_t at = 0xffffffffu;
#pragma unroll
    for (int i = 0; i < 8; i++) {
      const float a = fabsf(v[i]);
      if (a > amax) amax = a, mx = v[i], at = 8 * l32 + i;
    }
#pragma unroll
    for (int o = 16; o > 0; o >>= 1) {
      const float oa = __shfl_xor(amax, o, 32), om = __shfl_xor(mx, o, 32);
      const uint32_t oi = __shfl_xor(at, o, 32);
      if (oa > amax || (oa == amax && oi < at)) amax = oa, mx = om, at = oi;
    }
    float d = 0.0f;
    int part = 0;
    if (amax != 0.0f) {
      const float iscale = __fdiv_rn(-127.0f, mx);
#pragma unroll
      for (int i = 0; i < 8; i++) {
        int q = nearest_int(__fmul_rn(iscale, v[i]));
        q = q < 127 ? q : 127;
        part += q;
        code[i / 4] |= ((uint32_t)q & 0xffu) << (8 * (i % 4));
      }
      d = __fdiv_rn(1.0f, iscale);
    }
    part += __shfl_xor(part, 1, 32);
    part += __shfl_xor(part, 2, 32);
    ((uint2 *)out)[l32] = make_uint2(code[0], code[1]);
    if ((l32 & 3u) == 0) ((int32_t *)(out + kActSums))[l32 / 4] = part;
    if (l32 == 0) ((float *)(out + kActScales))[0] = d;
  } else {  // q8_0: blocks of 32, four lanes each
    float amax = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; i++) amax = fmaxf(amax, fabsf(v[i]));
    amax = fmaxf(amax, __shfl_xor(amax, 1, 32));
    amax = fmaxf(amax, __shfl_xor(amax, 2, 32));
    const float d = __fdiv_rn(amax, 127.0f), id = amax != 0.0f ? __fdiv_rn(127.0f, amax) : 0.0f;
#pragma unroll
    for (int i = 0; i < 8; i++) {
      const int q = nearest_int(__fmul_rn(v[i], id));
      code[i / 4] |= ((uint32_t)q & 0xffu) << (8 * (i % 4));
    }
    ((uint2 *)out)[l32] = make_uint2(code[0], code[1]);
    if ((l32 & 3u) == 0) ((float *)(out + kActScales))[l32 / 4] = h2f(f2h(d));
    if ((l32 & 3u) == 0) ((int32_t *)(out + kActSums))[l32 / 4] = 0;
  }
}

__device__ __forceinline__ uint64_t order_key(float logit, uint32_t id) {
  uint32_t u = __float_as_uint(__fadd_rn(logit, 0.0f));  // -0 as +0
  u ^= (u >> 31) ? 0xffffffffu : 0x80000000u;             // larger float, larger key
  return ((uint64_t)u << 32) | (0xffffffffu - id);        // equal logits: the lower id is larger
}

// Top-k, weights and the shared gate for token t, by one wave.
__device__ void route_token(const DecodeParams &p, uint32_t t, int32_t *ids_lds) {
  const uint32_t lane = lane_id(), E = p.E, K = p.K;
  const float *lg = p.logits + (uint64_t)t * (E + 1);
  constexpr int kPer = kMaxExperts / 64;
  float v[kPer];
  float mx = -INFINITY;
#pragma unroll
  for (int i = 0; i < kPer; i++) {
    const uint32_t e = lane + 64 * i;
    v[i] = e < E ? ld_co(lg + e) : -INFINITY;
    mx = fmaxf(mx, v[i]);
  }
  mx = wave_max(mx);
  double sum = 0.0;
#pragma unroll
  for (int i = 0; i < kPer; i++)
    if (lane + 64 * i < E) sum = __dadd_rn(sum, (double)expf_libm(__fsub_rn(v[i], mx)));
  sum = wave_sum_d(sum);
  const float inv = (float)(1.0 / sum);
  bool taken[kPer];
#pragma unroll
  for (int i = 0; i < kPer; i++) taken[i] = lane + 64 * i >= E;
  uint32_t my_id = 0;
  float my_l = 0.0f;
  for (uint32_t r = 0; r < K; r++) {
    uint64_t best = 0;
    int bi = -1;
#pragma unroll
    for (int i = 0; i < kPer; i++) {
      if (taken[i]) continue;
      const uint64_t key = order_key(v[i], lane + 64 * i);
      if (bi < 0 || key > best) best = key, bi = i;
    }
    uint64_t wbest = best;
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
      const uint64_t other = __shfl_xor(wbest, o, 64);
      wbest = other > wbest ? other : wbest;
    }
    const uint32_t wid = 0xffffffffu - (uint32_t)wbest;
    if (bi >= 0 && best == wbest) taken[bi] = true;
    if (lane == r) {  // the logit back from its key
      const uint32_t k = (uint32_t)(wbest >> 32);
      my_id = wid;
      my_l = __uint_as_float((k & 0x80000000u) ? (k ^ 0x80000000u) : ~k);
    }
  }
  const float pk = lane < K ? __fmul_rn(expf_libm(__fsub_rn(my_l, mx)), inv) : 0.0f;
  float tot = 0.0f;
  for (uint32_t r = 0; r < K; r++) tot = __fadd_rn(tot, __shfl(pk, r, 64));
  const float den = fmaxf(tot, 6.1035e-5f);
  if (lane < K) {
    p.ids[t * K + lane] = (int32_t)my_id;
    p.w[t * K + lane] = __fdiv_rn(pk, den);
    ids_lds[t * K + lane] = (int32_t)my_id;
  }
  if (lane == 0) p.gs[t] = sigmoid_libm(ld_co(lg + E));
}

}  // namespace

// Grid: max(ceil((E + 1) / 16), T) work-groups of 512. Work-group b < T quantises token b; every work-group takes 16
// router rows (2 a wave); the last one to finish routes every token (a wave a token) and groups the assignments.
__global__ void __launch_bounds__(kRouteWG) moe_route(DecodeParams p) {
  __shared__ int32_t ids_lds[kMaxDecodeTokens * kMaxUsed];
  __shared__ uint32_t s_head[kRouteWG], s_flag;
  __shared__ double part[kRouteWG / 64][2 * kMaxDecodeTokens][64];
  const uint32_t lane = lane_id(), wave = wave_id(), H = p.H, E = p.E, K = p.K, T = p.T;
  if (blockIdx.x < T) {
    // x[t] to the activation types of the routed and the shared gate: a half-wave per unit.
    const uint32_t t = blockIdx.x, l32 = threadIdx.x & 31u;
    for (uint32_t u = threadIdx.x / 32; u < H / kUnit; u += kRouteWG / 32) {
      float v[8];
      const float4 *src = (const float4 *)(p.x + (uint64_t)t * H + u * kUnit + 8 * l32);
      const float4 a = src[0], b = src[1];
      v[0] = a.x, v[1] = a.y, v[2] = a.z, v[3] = a.w, v[4] = b.x, v[5] = b.y, v[6] = b.z, v[7] = b.w;
      quant_unit(v, l32, p.xact_r, p.act_r + ((uint64_t)t * (H / kUnit) + u) * kActBytes);
      if (p.act_s != p.act_r) quant_unit(v, l32, p.xact_s, p.act_s + ((uint64_t)t * (H / kUnit) + u) * kActBytes);
    }
  }
  if (!p.route) return;
  // Router rows: logit = sum of bf16(W) bf16(x), products exact, summed in fp64, rounded once, plus the bias. A lane
  // keeps one fp64 partial per (row, token); the wave then sums each pair's 64 partials through LDS.
  const uint32_t r0 = blockIdx.x * 16 + wave * 2, npair = 2 * T;
  for (uint32_t rr = 0; rr < 2; rr++) {
    const uint32_t r = r0 + rr;
    const uint16_t *wr = p.router + (uint64_t)(r <= E ? r : E) * H;
    for (uint32_t t = 0; t < T; t++) {
      const float *xt = p.x + (uint64_t)t * H;
      double acc = 0.0;
      for (uint32_t c = lane * 8; c < H; c += 512) {
        const uint4 wv = *(const uint4 *)(wr + c);
        const float4 x0 = *(const float4 *)(xt + c), x1 = *(const float4 *)(xt + c + 4);
        const uint32_t ww[4] = {wv.x, wv.y, wv.z, wv.w};
        const float xx[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
#pragma unroll
        for (int i = 0; i < 8; i++) {
          const float wf = bf2f((uint16_t)(ww[i / 2] >> (16 * (i % 2))));
          acc = __builtin_fma((double)wf, (double)round_bf16(xx[i]), acc);
        }
      }
      part[wave][rr * T + t][lane] = acc;
    }
  }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
  __builtin_amdgcn_wave_barrier();
  {
    uint32_t lp = 64;  // lanes per pair: 64 / the next power of two of npair
    while (lp > 1 && (64 / lp) < npair) lp /= 2;
    const uint32_t pr = lane / lp, q = lane % lp, span = 64 / lp;
    double acc = 0.0;
    if (pr < npair)
      for (uint32_t i = 0; i < span; i++) acc = __dadd_rn(acc, part[wave][pr][q * span + i]);
    for (uint32_t o = 1; o < lp; o <<= 1) acc = __dadd_rn(acc, __shfl_xor(acc, o, 64));
    const uint32_t r = r0 + pr / T, t = pr % T;
    if (pr < npair && q == 0 && r <= E) {
      float l = (float)acc;
      if (r < E && p.bias) l = __fadd_rn(l, p.bias[r]);
      st_co(p.logits + (uint64_t)t * (E + 1) + r, l);
    }
  }
  if (!arrive_last(p.cnt_route, gridDim.x, &s_flag)) return;
  for (uint32_t t = wave; t < T; t += kRouteWG / 64) route_token(p, t, ids_lds);
  __syncthreads();
  // MoeGroup records: an expert's assignments in order, MOE_GROUP_MAX a group, groups numbered by their first
  // assignment (as group_slots, layer.cl:894-942), then the shared expert's groups.
  const uint32_t n = T * K, a = threadIdx.x;
  int32_t e = -1;
  uint32_t rank = 0, total = 0, head_rank = 0, head_a = 0;
  if (a < n) {
    e = ids_lds[a];
    for (uint32_t b = 0; b < n; b++)
      if (ids_lds[b] == e) {
        if (b < a) rank++;
        total++;
      }
    head_rank = rank - rank % MOE_GROUP_MAX;
    for (uint32_t b = 0, seen = 0; b <= a; b++)
      if (ids_lds[b] == e) {
        if (seen == head_rank) {
          head_a = b;
          break;
        }
        seen++;
      }
  }
  const bool head = a < n && rank % MOE_GROUP_MAX == 0;
  s_head[a] = head ? 1u : 0u;
  __syncthreads();
  for (uint32_t off = 1; off < kRouteWG; off <<= 1) {  // inclusive scan of the heads
    const uint32_t add = a >= off ? s_head[a - off] : 0u;
    __syncthreads();
    s_head[a] += add;
    __syncthreads();
  }
  const uint32_t nr = s_head[kRouteWG - 1];
  if (a < n) {
    const uint32_t g = s_head[head_a] - 1;
    p.groups[g].asg[rank % MOE_GROUP_MAX] = a;
    if (head) {
      p.groups[g].slot = e;
      p.groups[g].n = min((uint32_t)MOE_GROUP_MAX, total - rank);
    }
  }
  const uint32_t ns = p.has_shared ? (T + MOE_GROUP_MAX - 1) / MOE_GROUP_MAX : 0;
  if (a < ns) {
    p.groups[nr + a].slot = (int32_t)E;
    p.groups[nr + a].n = min((uint32_t)MOE_GROUP_MAX, T - a * MOE_GROUP_MAX);
    for (uint32_t j = 0; j < MOE_GROUP_MAX; j++)
      if (a * MOE_GROUP_MAX + j < T) p.groups[nr + a].asg[j] = n + a * MOE_GROUP_MAX + j;
  }
  if (a == 0) *p.ngroups = nr + ns;
}

namespace {

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

__device__ __forceinline__ void load_grid(uint32_t *grid_lds, uint32_t nthreads) {
  for (uint32_t i = threadIdx.x; i < 512; i += nthreads) grid_lds[i] = kIq3sGridDev[i];
}

// The n terms of one (row, unit) pair against the activation units act + j * kActLds / 4 dwords, into t[j].
__device__ __forceinline__ void pair_terms(uint32_t type, const uint8_t *tile, uint32_t idx, uint32_t nl,
                                           const uint32_t *grid_lds, const uint32_t *act, uint32_t stride, uint32_t n,
                                           float *t) {
  switch (type) {
    case QT_Q8_0: {
      UnitQ8_0 w;
      w.load(tile, idx, nl);
      #pragma unroll
      for (uint32_t j = 0; j < MOE_GROUP_MAX; j++)
        if (j < n) t[j] = w.term(Act(act + j * stride));
      break;
    }
    case QT_Q4_K: {
      UnitQ4_K w;
      w.load(tile, idx, nl);
      #pragma unroll
      for (uint32_t j = 0; j < MOE_GROUP_MAX; j++)
        if (j < n) t[j] = w.term(Act(act + j * stride));
      break;
    }
    default: {
      UnitIQ3_S w;
      w.load(tile, idx, nl, grid_lds);
      #pragma unroll
      for (uint32_t j = 0; j < MOE_GROUP_MAX; j++)
        if (j < n) t[j] = w.term(Act(act + j * stride));
      break;
    }
  }
}

// The pairwise sum over the U lanes of a row (U a power of two, the lanes consecutive): butterflies, which add the
// halves in the oracle's tree order.
__device__ __forceinline__ float row_sum(float t, uint32_t U) {
  for (uint32_t o = 1; o < U; o <<= 1) t = __fadd_rn(t, __shfl_xor(t, o, 64));
  return t;
}

}  // namespace

// Grid: G_max x (F / gate_up_rows(U)) work-groups of 256. A work-group takes gate_up_rows rows of gate and of up of
// group g's expert, all U units of each: lane = m * 32 + r * U + u (m gate or up, r a row of the wave's 32 / U).
// Each row's units are summed inside the wave, so h = silu(g) * u is whole here and stored as fp32.
__global__ void __launch_bounds__(kGateUpWG) moe_gate_up(DecodeParams p) {
  extern __shared__ uint32_t dyn_lds[];  // the group's activation units, kActLds apart
  __shared__ uint32_t grid_lds[512];
  const uint32_t U = p.H / kUnit, rows = gate_up_rows(U), nwg = p.F / rows;
  const uint32_t g = blockIdx.x / nwg, row0 = (blockIdx.x % nwg) * rows;
  if (g >= *p.ngroups) return;
  const MoeGroup &grp = p.groups[g];
  const uint32_t n = grp.n;
  const GroupMat gm = group_mat(p, grp.slot, 0);
  const uint8_t *act = gm.shared ? p.act_s : p.act_r;
  // Stage the n assignments' activation units (their tokens' x, quantised by moe_route).
  for (uint32_t i = threadIdx.x; i < n * U * (kActBytes / 16); i += kGateUpWG) {
    const uint32_t unit = i / (kActBytes / 16), c = i % (kActBytes / 16), j = unit / U, u = unit % U;
    const uint4 v = ((const uint4 *)(act + ((uint64_t)asg_token(p, grp.asg[j]) * U + u) * kActBytes))[c];
    *(uint4 *)((uint8_t *)dyn_lds + unit * kActLds + 16 * c) = v;
  }
  if (gm.type == QT_IQ3_S) load_grid(grid_lds, kGateUpWG);
  __syncthreads();
  const uint32_t lane = lane_id(), m = lane / 32, r = (lane % 32) / U, u = lane % U;
  const uint32_t row = row0 + wave_id() * (32 / U) + r;
  const uint8_t *mat = gm.mat + (m ? (gm.shared ? p.sh_up_off : p.ex_up_off) : 0);
  const uint8_t *tile = mat + (uint64_t)(row / kTileRows) * tile_bytes(gm.type, U);
  float t[MOE_GROUP_MAX];
  pair_terms(gm.type, tile, (row % kTileRows) * U + u, kTileRows * U, grid_lds, dyn_lds + u * (kActLds / 4),
             U * (kActLds / 4), n, t);
#pragma unroll
  for (uint32_t j = 0; j < MOE_GROUP_MAX; j++) {
    if (j >= n) break;
    const float s = row_sum(t[j], U);                 // gate's row sum in lanes m = 0, up's in m = 1
    const float su = __shfl_xor(s, 32, 64);           // the other matrix's
    if (m == 0 && u == 0) p.h[(uint64_t)grp.asg[j] * p.F + row] = swiglu_one(s, su, p.swiglu_limit);
  }
}

// Grid: G_max x (H / down_rows(Ud)) work-groups of 128. A work-group first quantises its group's h (each assignment's
// F values, as units of the down's activation type) into LDS, then takes down_rows rows of down, all Ud units:
// lane = r * Ud + u. A row's units are summed inside the wave into the assignment's output; a token whose k + 1
// outputs are all in for these rows is combined by the work-group that brought the last.
__global__ void __launch_bounds__(kDownWG) moe_down(DecodeParams p) {
  extern __shared__ uint32_t dyn_lds[];
  __shared__ uint32_t grid_lds[512];
  __shared__ uint32_t s_last[MOE_GROUP_MAX];
  const uint32_t U = p.F / kUnit, rows = down_rows(U), nwg = p.H / rows;
  const uint32_t g = blockIdx.x / nwg, rb = blockIdx.x % nwg, row0 = rb * rows;
  if (g >= *p.ngroups) return;
  const MoeGroup &grp = p.groups[g];
  const uint32_t n = grp.n;
  const GroupMat gm = group_mat(p, grp.slot, 2);
  const uint32_t dact = quant_vec_dot_type(gm.type);
  // h -> activation units in LDS: a half-wave a unit.
  for (uint32_t unit = threadIdx.x / 32; unit < n * U; unit += kDownWG / 32) {
    const uint32_t j = unit / U, u = unit % U, l32 = threadIdx.x & 31u;
    const float4 *src = (const float4 *)(p.h + (uint64_t)grp.asg[j] * p.F + u * kUnit + 8 * l32);
    const float4 a = src[0], b = src[1];
    const float v[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
    quant_unit(v, l32, dact, (uint8_t *)dyn_lds + unit * kActLds);
  }
  if (gm.type == QT_IQ3_S) load_grid(grid_lds, kDownWG);
  __syncthreads();
  const uint32_t lane = lane_id(), r = lane / U, u = lane % U;
  const uint32_t row = row0 + wave_id() * (64 / U) + r;
  const uint8_t *tile = gm.mat + (uint64_t)(row / kTileRows) * tile_bytes(gm.type, U);
  float t[MOE_GROUP_MAX];
  pair_terms(gm.type, tile, (row % kTileRows) * U + u, kTileRows * U, grid_lds, dyn_lds + u * (kActLds / 4),
             U * (kActLds / 4), n, t);
#pragma unroll
  for (uint32_t j = 0; j < MOE_GROUP_MAX; j++) {
    if (j >= n) break;
    const float s = row_sum(t[j], U);
    if (u == 0) st_co(p.y_asg + (uint64_t)grp.asg[j] * p.H + row, s);
  }
  // Count this work-group's outputs in, one counter per (token, row block), all at once.
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (threadIdx.x < n) {
    const uint32_t tk = asg_token(p, grp.asg[threadIdx.x]);
    const uint32_t need = p.tok_need ? p.tok_need[tk] : p.K + (p.has_shared ? 1u : 0u);
    uint32_t *cnt = p.cnt_tok + (uint64_t)tk * nwg + rb;
    const uint32_t old = __hip_atomic_fetch_add(cnt, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    s_last[threadIdx.x] = old == need - 1;
    if (old == need - 1) __hip_atomic_store(cnt, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  __syncthreads();
  // y = sum_k w_k y_k in rank order, then + gs s: every output loaded first, then summed in order.
  for (uint32_t j = 0; j < n; j++) {
    if (!s_last[j]) continue;
    const uint32_t tk = asg_token(p, grp.asg[j]);
    for (uint32_t i = threadIdx.x; i < rows; i += kDownWG) {
      const uint32_t rr = row0 + i;
      float yv[kMaxUsed + 1], wv[kMaxUsed];
      bool on[kMaxUsed];
#pragma unroll
      for (uint32_t k = 0; k < kMaxUsed; k++) {
        on[k] = k < p.K && p.ids[tk * p.K + k] >= 0;
        wv[k] = k < p.K ? p.w[tk * p.K + k] : 0.0f;
        yv[k] = on[k] ? ld_co(p.y_asg + ((uint64_t)tk * p.K + k) * p.H + rr) : 0.0f;
      }
      yv[kMaxUsed] = p.has_shared ? ld_co(p.y_asg + ((uint64_t)p.T * p.K + tk) * p.H + rr) : 0.0f;
      float acc = 0.0f;
#pragma unroll
      for (uint32_t k = 0; k < kMaxUsed; k++)
        if (on[k]) acc = __fadd_rn(acc, __fmul_rn(wv[k], yv[k]));
      if (p.has_shared) acc = __fadd_rn(acc, __fmul_rn(p.gs[tk], yv[kMaxUsed]));
      p.y[(uint64_t)tk * p.H + rr] = acc;
    }
  }
}

}  // namespace c0ven
