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

__device__ __forceinline__ void route_load(const float *lg, uint32_t E, uint32_t lane, uint32_t key[kRoutePer],
                                           uint32_t id[kRoutePer]) {
#pragma unroll
  for (int i = 0; i < kRoutePer; i++) {
    const uint32_t e = lane + 64 * i;
    key[i] = e < E ? float_key(ld_co(lg + e)) : 0u;
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

// Lane r < K's renormalised weight (the whole wave takes part).
__device__ __forceinline__ float route_weight(uint32_t my_key, float mx, float inv, uint32_t K, uint32_t lane,
                                              const uint64_t *tab) {
  const float pk = lane < K ? __fmul_rn(expf_libm(__fsub_rn(key_float(my_key), mx), tab), inv) : 0.0f;
  float tot = 0.0f;
  for (uint32_t r = 0; r < K; r++) tot = __fadd_rn(tot, __uint_as_float(readlane_u32(__float_as_uint(pk), r)));
  return __fdiv_rn(pk, fmaxf(tot, 6.1035e-5f));
}

}  // namespace c0ven
