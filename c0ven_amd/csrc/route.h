// The router's per-token steps as wave-level pieces (route.h:39-99 and layer.cl:765-804 of the reference restated),
// shared by the decode kernel (two waves per token) and the prefill top-k kernel (one wave per token).
//
// Lane l holds experts l + 64 i (i < 8) as order keys of their logits (float_key: -0 as +0). The softmax takes the
// max and sum_e expf(l_e - max) in double; P_k = expf(l_k - max) * (float)(1 / sum). The top k are by logit with the
// lower id first among equal logits; w_k = P_k / max(sum of the k P in rank order, 6.1035e-5).
#pragma once

#include "act_quant.h"
#include "device_math.h"

namespace c0ven {

constexpr int kRoutePer = 8;  // experts a lane holds (512 / 64)

// kCoherent: the logits were written by other work-groups of the same launch (an L2-coherent load); otherwise by an
// earlier kernel (a plain load).
template <bool kCoherent = true>
__device__ __forceinline__ void route_load(const float *lg, uint32_t E, uint32_t lane, uint32_t key[kRoutePer],
                                           uint32_t id[kRoutePer]) {
#pragma unroll
  for (int i = 0; i < kRoutePer; i++) {
    const uint32_t e = lane + 64 * i;
    key[i] = e < E ? float_key(kCoherent ? ld_co(lg + e) : lg[e]) : 0u;
    id[i] = e;
  }
}

// The softmax's max and 1 / sum (wave-uniform).
__device__ __forceinline__ void route_norm(const uint32_t key[kRoutePer], uint32_t E, uint32_t lane,
                                           const uint64_t *tab, float *mx_out, float *inv_out) {
  uint32_t mk = 0;
#pragma unroll
  for (int i = 0; i < kRoutePer; i++) mk = max(mk, key[i]);
  const float mx = key_float(wave_max_u32(mk));
  double part = 0.0;
#pragma unroll
  for (int i = 0; i < kRoutePer; i++)
    if (lane + 64 * i < E) part = __dadd_rn(part, (double)expf_libm(__fsub_rn(key_float(key[i]), mx), tab));
  const double sum = wave_sum_f64(part);
  *mx_out = mx;
  *inv_out = (float)(1.0 / sum);
}

// The softmax's max (wave-uniform) from a lane's keys.
__device__ __forceinline__ float route_max(const uint32_t key[kRoutePer]) {
  uint32_t mk = 0;
#pragma unroll
  for (int i = 0; i < kRoutePer; i++) mk = max(mk, key[i]);
  return key_float(wave_max_u32(mk));
}

// Part `part` (0, 1 or 2) of the softmax's sum: the wave's double sum of expf(l_e - mx) over the lane slots
// i = part, part + 3, ... (the three parts together cover every expert once).
__device__ __forceinline__ double route_sum_part(const uint32_t key[kRoutePer], uint32_t E, uint32_t lane, uint32_t part,
                                                 float mx, const uint64_t *tab) {
  double acc = 0.0;
#pragma unroll
  for (int k = 0; k < 3; k++) {
    const uint32_t i = part + 3 * k;  // wave-uniform; the select keeps the key in a register
    // Masks rather than a select of array elements, which the compiler would turn into an indexed (scratch) load.
    const uint32_t m0 = 0u - (uint32_t)(part == 0), m1 = 0u - (uint32_t)(part == 1), m2 = 0u - (uint32_t)(part == 2);
    const uint32_t kk = (key[3 * k] & m0) | (key[(3 * k + 1) % kRoutePer] & m1) | (key[(3 * k + 2) % kRoutePer] & m2);
    const float e = expf_libm(__fsub_rn(key_float(kk), mx), tab);
    acc = __dadd_rn(acc, i < kRoutePer && lane + 64 * i < E ? (double)e : 0.0);
  }
  return wave_sum_f64(acc);
}

// The top K: lane r < K receives the r-th winner's id and key. Sorts each lane's keys, largest first (ids ascending
// within a lane, so equal keys keep the lower id first); each round takes the wave's largest head (a DPP max, a
// ballot for equal keys, the lower id among them) and pops it. key and id are consumed.
__device__ __forceinline__ void route_select(uint32_t key[kRoutePer], uint32_t id[kRoutePer], uint32_t K,
                                             uint32_t lane, uint32_t *my_id, uint32_t *my_key) {
  auto cswap = [&](int i, int j) {
    const bool sw = (key[j] > key[i]) | ((key[j] == key[i]) & (id[j] < id[i]));  // no short circuit: no branches
    const uint32_t ki = key[i], ii = id[i];
    key[i] = sw ? key[j] : ki, id[i] = sw ? id[j] : ii;
    key[j] = sw ? ki : key[j], id[j] = sw ? ii : id[j];
  };
  cswap(0, 1), cswap(2, 3), cswap(4, 5), cswap(6, 7), cswap(0, 2), cswap(1, 3), cswap(4, 6), cswap(5, 7);
  cswap(1, 2), cswap(5, 6), cswap(0, 4), cswap(3, 7), cswap(1, 5), cswap(2, 6), cswap(1, 4), cswap(3, 6);
  cswap(2, 4), cswap(3, 5), cswap(3, 4);
  uint32_t mi = 0, mk = 0;
  for (uint32_t r = 0; r < K; r++) {
    const uint32_t m = wave_max_u32(key[0]);
    const uint64_t cand = __ballot(key[0] == m);
    uint32_t wid;
    if (__popcll(cand) == 1) {
      wid = readlane_u32(id[0], __ffsll((long long)cand) - 1);
    } else {
      wid = wave_min_u32(key[0] == m ? id[0] : 0xffffffffu);
    }
    if (lane == r) mi = wid, mk = m;
    if (key[0] == m && id[0] == wid) {  // pop the winner
#pragma unroll
      for (int i = 0; i < kRoutePer - 1; i++) key[i] = key[i + 1], id[i] = id[i + 1];
      key[kRoutePer - 1] = 0;
    }
  }
  *my_id = mi, *my_key = mk;
}

// The top K as route_select gives them (same winners, same order), by a threshold instead of K rounds: tau, the K-th
// largest of the lanes' maxima, is found bit by bit with ballots; at least K keys are >= tau (one a lane of those K
// lanes), so every winner is among the keys >= tau. Those candidates (usually little more than K) are packed into
// cand (LDS, room for 64 kRoutePer + K entries) and each is ranked against all of them: rank = the number that beat it
// (a larger key, or an equal key with a lower id): with at most 64 candidates in registers (each lane reads the others
// with readlane), otherwise in LDS. One wave runs this; key and id are kept.
__device__ __forceinline__ void route_select_lds(const uint32_t key[kRoutePer], const uint32_t id[kRoutePer], uint32_t K,
                                                 uint32_t lane, uint2 *cand, uint32_t *my_id, uint32_t *my_key) {
  uint32_t m = key[0];
#pragma unroll
  for (int i = 1; i < kRoutePer; i++) m = max(m, key[i]);
  uint32_t tau = 0;
  for (int b = 31; b >= 0; b--) {
    const uint32_t c = tau | (1u << b);
    if ((uint32_t)__popcll(__ballot(m >= c)) >= K) tau = c;
  }
  uint32_t cnt = 0;
#pragma unroll
  for (int i = 0; i < kRoutePer; i++) cnt += key[i] >= tau ? 1u : 0u;
  uint32_t pos = 0, total = 0;  // this lane's first slot (the counts of the lanes below it) and the wave's count
#pragma unroll
  for (int b = 0; b < 4; b++) {
    const uint64_t bal = __ballot((cnt >> b) & 1u);
    pos += __builtin_amdgcn_mbcnt_hi((uint32_t)(bal >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)bal, 0u)) << b;
    total += (uint32_t)__popcll(bal) << b;
  }
#pragma unroll
  for (int i = 0; i < kRoutePer; i++) {
    if (key[i] >= tau) cand[pos] = make_uint2(key[i], id[i]);
    pos += key[i] >= tau ? 1u : 0u;
  }
  __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): this wave's LDS stores are done before it reads them back
  __builtin_amdgcn_wave_barrier();
  if (total <= 64) {  // (the usual case) candidate j in lane j, ranked against the others read lane by lane
    const uint2 me = lane < total ? cand[lane] : make_uint2(0u, 0u);
    uint32_t rank = 0;
    for (uint32_t i = 0; i < total; i++) {
      const uint32_t ok = readlane_u32(me.x, (int)i), oi = readlane_u32(me.y, (int)i);
      rank += (ok > me.x) | ((ok == me.x) & (oi < me.y));
    }
    // Ranks of the candidates are distinct and below total; the other lanes keep their own index: a permutation, so
    // one ds_permute (lane rank receives the candidate of that rank) moves every winner to its lane.
    const int dst = 4 * (int)(lane < total ? rank : lane);
    *my_key = (uint32_t)__builtin_amdgcn_ds_permute(dst, (int)me.x);
    *my_id = (uint32_t)__builtin_amdgcn_ds_permute(dst, (int)me.y);
    if (lane >= K) *my_key = 0u, *my_id = 0u;
    return;
  }
  uint2 *sel = cand + 64 * kRoutePer;
  for (uint32_t j = lane; j < total; j += 64) {
    const uint2 me = cand[j];
    uint32_t rank = 0;
    for (uint32_t i = 0; i < total; i++) {
      const uint2 o = cand[i];
      rank += (o.x > me.x) | ((o.x == me.x) & (o.y < me.y));
    }
    if (rank < K) sel[rank] = me;
  }
  __builtin_amdgcn_s_waitcnt(0xc07f);
  __builtin_amdgcn_wave_barrier();
  const uint2 w = lane < K ? sel[lane] : make_uint2(0u, 0u);
  *my_key = w.x, *my_id = w.y;
}

// Lane r < K's renormalised weight (the whole wave takes part).
__device__ __forceinline__ float route_weight(uint32_t my_key, float mx, float inv, uint32_t K, uint32_t lane,
                                              const uint64_t *tab) {
  const float pk = lane < K ? __fmul_rn(expf_libm(__fsub_rn(key_float(my_key), mx), tab), inv) : 0.0f;
  float tot = 0.0f;
  for (uint32_t r = 0; r < K; r++) tot = __fadd_rn(tot, __uint_as_float(readlane_u32(__float_as_uint(pk), r)));
  return __fdiv_rn(pk, fmaxf(tot, 6.1035e-5f));
}

}  // namespace c0ven
