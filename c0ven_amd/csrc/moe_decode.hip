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

constexpr uint32_t kWG = 256;  // threads of every decode work-group: four waves

__device__ __forceinline__ uint32_t lane_id() { return threadIdx.x & 63u; }
__device__ __forceinline__ uint32_t wave_id() { return threadIdx.x >> 6; }

// Counts the work-group in on *cnt after its writes; true in every thread of the one that completes `total`.
__device__ __forceinline__ bool arrive_last(uint32_t *cnt, uint32_t total, uint32_t *flag) {
  __threadfence();
  __syncthreads();
  if (threadIdx.x == 0) {
    const uint32_t old = atomicAdd(cnt, 1u);
    *flag = old == total - 1;
    if (old == total - 1) atomicExch(cnt, 0u);
  }
  __syncthreads();
  const bool last = *flag != 0;
  if (last) __threadfence();
  return last;
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
    v[i] = e < E ? lg[e] : -INFINITY;
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
    if (lane == r) {
      my_id = wid;
      my_l = lg[wid];
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
  if (lane == 0) p.gs[t] = sigmoid_libm(lg[E]);
}

}  // namespace

// Grid: max(ceil((E + 1) / 8), T) work-groups of 256. Work-group b < T quantises token b; every work-group takes 8
// router rows (2 a wave); the last one to finish routes every token and groups the assignments.
__global__ void __launch_bounds__(kWG) moe_route(DecodeParams p) {
  __shared__ int32_t ids_lds[kMaxDecodeTokens * kMaxUsed];
  __shared__ uint32_t s_head[kWG], s_flag;
  const uint32_t lane = lane_id(), wave = wave_id(), H = p.H, E = p.E, K = p.K, T = p.T;
  if (blockIdx.x < T) {
    // x[t] to the activation types of the routed and the shared gate: a half-wave per unit.
    const uint32_t t = blockIdx.x, l32 = threadIdx.x & 31u;
    for (uint32_t u = threadIdx.x / 32; u < H / kUnit; u += kWG / 32) {
      float v[8];
      const float4 *src = (const float4 *)(p.x + (uint64_t)t * H + u * kUnit + 8 * l32);
      const float4 a = src[0], b = src[1];
      v[0] = a.x, v[1] = a.y, v[2] = a.z, v[3] = a.w, v[4] = b.x, v[5] = b.y, v[6] = b.z, v[7] = b.w;
      quant_unit(v, l32, p.xact_r, p.act_r + ((uint64_t)t * (H / kUnit) + u) * kActBytes);
      if (p.act_s != p.act_r) quant_unit(v, l32, p.xact_s, p.act_s + ((uint64_t)t * (H / kUnit) + u) * kActBytes);
    }
  }
  if (!p.route) return;
  // Router rows: logit = sum of bf16(W) bf16(x), products exact, summed in fp64, rounded once, plus the bias.
  for (uint32_t rr = 0; rr < 2; rr++) {
    const uint32_t r = blockIdx.x * 8 + wave * 2 + rr;
    if (r > E) break;
    const uint16_t *wr = p.router + (uint64_t)r * H;
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
      acc = wave_sum_d(acc);
      if (lane == 0) {
        float l = (float)acc;
        if (r < E && p.bias) l = __fadd_rn(l, p.bias[r]);
        p.logits[(uint64_t)t * (E + 1) + r] = l;
      }
    }
  }
  if (!arrive_last(p.cnt_route, gridDim.x, &s_flag)) return;
  for (uint32_t t = wave; t < T; t += kWG / 64) route_token(p, t, ids_lds);
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
  for (uint32_t off = 1; off < kWG; off <<= 1) {  // inclusive scan of the heads
    const uint32_t add = a >= off ? s_head[a - off] : 0u;
    __syncthreads();
    s_head[a] += add;
    __syncthreads();
  }
  const uint32_t nr = s_head[kWG - 1];
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

// The tile (64 rows of one unit) a wave reads, and the matrix's type, for group g's expert.
struct GroupMat {
  const uint8_t *mat;
  uint32_t type;
  bool shared;
};

__device__ __forceinline__ GroupMat group_mat(const DecodeParams &p, const MoeGroup &g, int which) {
  GroupMat m;
  m.shared = g.slot == (int32_t)p.E;
  if (m.shared) {
    m.type = which == 2 ? p.sh_down_type : p.sh_gate_type;
    m.mat = p.shared + (which == 0 ? 0 : which == 1 ? p.sh_up_off : p.sh_down_off);
  } else {
    m.type = which == 2 ? p.down_type : p.gate_type;
    m.mat = p.experts + (uint64_t)g.slot * p.ex_bytes + (which == 0 ? 0 : which == 1 ? p.ex_up_off : p.ex_down_off);
  }
  return m;
}

__device__ __forceinline__ uint32_t asg_token(const DecodeParams &p, uint32_t asg) {
  const uint32_t n = p.T * p.K;
  return asg < n ? asg / p.K : asg - n;
}

// The terms of one tile against the n activation units act(j), into out[j * stride].
template <typename Act>
__device__ __forceinline__ void tile_terms(uint32_t type, const uint8_t *tile, const uint32_t *grid_lds, uint32_t n,
                                           Act act, float *out, uint64_t stride) {
  const uint32_t lane = lane_id();
  switch (type) {
    case QT_Q8_0: {
      UnitQ8_0 w;
      w.load(tile, lane);
      for (uint32_t j = 0; j < n; j++) out[j * stride] = w.term(ActUnit(act(j)));
      break;
    }
    case QT_Q4_K: {
      UnitQ4_K w;
      w.load(tile, lane);
      for (uint32_t j = 0; j < n; j++) out[j * stride] = w.term(ActUnit(act(j)));
      break;
    }
    default: {
      UnitIQ3_S w;
      w.load(tile, lane, grid_lds);
      for (uint32_t j = 0; j < n; j++) out[j * stride] = w.term(ActUnit(act(j)));
      break;
    }
  }
}

__device__ __forceinline__ void load_grid(uint32_t *grid_lds) {
  for (uint32_t i = threadIdx.x; i < 512; i += kWG) grid_lds[i] = kIq3sGridDev[i];
  __syncthreads();
}

}  // namespace

// Grid: G_max x (F / 256) x 2 x (H / 256) work-groups of 256 (group slowest, then 256-row block, matrix, unit).
__global__ void __launch_bounds__(kWG) moe_gate_up(DecodeParams p) {
  __shared__ uint32_t grid_lds[512];
  __shared__ float hbuf[MOE_GROUP_MAX][kUnit];
  __shared__ uint32_t s_flag;
  const uint32_t Ug = p.H / kUnit, nrb = p.F / kUnit;
  uint32_t wg = blockIdx.x;
  const uint32_t u = wg % Ug;
  wg /= Ug;
  const uint32_t m = wg % 2;
  wg /= 2;
  const uint32_t rb = wg % nrb, g = wg / nrb;
  if (g >= *p.ngroups) return;
  const MoeGroup grp = p.groups[g];
  const GroupMat gm = group_mat(p, grp, (int)m);
  if (gm.type == QT_IQ3_S) load_grid(grid_lds);
  const uint8_t *act = gm.shared ? p.act_s : p.act_r;
  const uint32_t row = rb * kUnit + threadIdx.x;  // wave w holds rows rb * 256 + 64 w + lane
  const uint8_t *tile = gm.mat + ((uint64_t)(rb * 4 + wave_id()) * Ug + u) * tile_bytes(gm.type);
  float *terms = p.terms_gu + (((uint64_t)g * 2 + m) * Ug + u) * MOE_GROUP_MAX * p.F + row;
  tile_terms(
      gm.type, tile, grid_lds, grp.n,
      [&](uint32_t j) { return act + ((uint64_t)asg_token(p, grp.asg[j]) * Ug + u) * kActBytes; }, terms, p.F);
  if (!arrive_last(p.cnt_gu + (uint64_t)g * nrb + rb, 2 * Ug, &s_flag)) return;
  // Finish rows rb * 256 .. +256: the units' pairwise sum, SwiGLU, h of each assignment quantised as one unit of the
  // down's K.
  const float *tg = p.terms_gu + ((uint64_t)g * 2 * Ug) * MOE_GROUP_MAX * p.F + row;
  const float *tu = tg + (uint64_t)Ug * MOE_GROUP_MAX * p.F;
  for (uint32_t j = 0; j < grp.n; j++) {
    float a[kMaxUnits], b[kMaxUnits];
    for (uint32_t k = 0; k < Ug; k++) {
      a[k] = tg[((uint64_t)k * MOE_GROUP_MAX + j) * p.F];
      b[k] = tu[((uint64_t)k * MOE_GROUP_MAX + j) * p.F];
    }
    hbuf[j][threadIdx.x] = swiglu_one(pairwise_pow2(a, Ug), pairwise_pow2(b, Ug), p.swiglu_limit);
  }
  __syncthreads();
  const uint32_t j = threadIdx.x / 32, l32 = threadIdx.x & 31u;
  if (j < grp.n) {
    float v[8];
#pragma unroll
    for (int i = 0; i < 8; i++) v[i] = hbuf[j][8 * l32 + i];
    const uint32_t dact = quant_vec_dot_type(group_mat(p, grp, 2).type);
    quant_unit(v, l32, dact, p.hact + ((uint64_t)grp.asg[j] * nrb + rb) * kActBytes);
  }
}

// Grid: G_max x (H / 256) x (F / 256) work-groups of 256 (group slowest, then 256-row block, unit).
__global__ void __launch_bounds__(kWG) moe_down(DecodeParams p) {
  __shared__ uint32_t grid_lds[512];
  __shared__ uint32_t s_flag;
  const uint32_t Ud = p.F / kUnit, nrb = p.H / kUnit;
  uint32_t wg = blockIdx.x;
  const uint32_t u = wg % Ud;
  wg /= Ud;
  const uint32_t rb = wg % nrb, g = wg / nrb;
  if (g >= *p.ngroups) return;
  const MoeGroup grp = p.groups[g];
  const GroupMat gm = group_mat(p, grp, 2);
  if (gm.type == QT_IQ3_S) load_grid(grid_lds);
  const uint32_t row = rb * kUnit + threadIdx.x;
  const uint8_t *tile = gm.mat + ((uint64_t)(rb * 4 + wave_id()) * Ud + u) * tile_bytes(gm.type);
  float *terms = p.terms_d + ((uint64_t)g * Ud + u) * MOE_GROUP_MAX * p.H + row;
  tile_terms(
      gm.type, tile, grid_lds, grp.n,
      [&](uint32_t j) { return p.hact + ((uint64_t)grp.asg[j] * Ud + u) * kActBytes; }, terms, p.H);
  if (!arrive_last(p.cnt_d + (uint64_t)g * nrb + rb, Ud, &s_flag)) return;
  const float *td = p.terms_d + (uint64_t)g * Ud * MOE_GROUP_MAX * p.H + row;
  for (uint32_t j = 0; j < grp.n; j++) {
    float a[kMaxUnits];
    for (uint32_t k = 0; k < Ud; k++) a[k] = td[((uint64_t)k * MOE_GROUP_MAX + j) * p.H];
    p.y_asg[(uint64_t)grp.asg[j] * p.H + row] = pairwise_pow2(a, Ud);
  }
  // A token whose k routed outputs and shared output are all in: y = sum_k w_k y_k (rank order) + gs s.
  for (uint32_t j = 0; j < grp.n; j++) {
    const uint32_t t = asg_token(p, grp.asg[j]);
    const uint32_t need = p.tok_need ? p.tok_need[t] : p.K + (p.has_shared ? 1u : 0u);
    if (!arrive_last(p.cnt_tok + (uint64_t)t * nrb + rb, need, &s_flag)) continue;
    const float *ya = p.y_asg + row;
    const float *wt = p.w + (uint64_t)t * p.K;
    const int32_t *it = p.ids + (uint64_t)t * p.K;
    float acc = 0.0f;
    for (uint32_t r = 0; r < p.K; r++)
      if (it[r] >= 0) acc = __fadd_rn(acc, __fmul_rn(wt[r], ya[((uint64_t)t * p.K + r) * p.H]));
    if (p.has_shared) acc = __fadd_rn(acc, __fmul_rn(p.gs[t], ya[((uint64_t)p.T * p.K + t) * p.H]));
    p.y[(uint64_t)t * p.H + row] = acc;
  }
}

}  // namespace c0ven
