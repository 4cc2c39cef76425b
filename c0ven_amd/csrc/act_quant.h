// Device-coherent accesses and the activation quantiser, shared by the decode and prefill kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/c0ven_quant.h"
#include "device_math.h"
#include "layout.h"

namespace c0ven {

// Data one work-group writes and another reads within a launch goes through device-coherent accesses (agent-scope
// relaxed atomics: the store writes through the XCD's L2, the load reads past a stale line), so no fence has to
// write back or invalidate a whole L2. Kernel boundaries order everything else.
template <typename T>
__device__ __forceinline__ void st_co(T *p, T v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
template <typename T>
__device__ __forceinline__ T ld_co(const T *p) {
  return __hip_atomic_load(const_cast<T *>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// A tagged record: a 32-bit value in the low word, the writing launch's tag in the high word, stored and loaded as one
// 64-bit access (single-copy atomic), so a reader that sees its launch's tag sees the value written with it.
__device__ __forceinline__ void st_tag(uint64_t *p, uint32_t v, uint32_t tag) {
  __hip_atomic_store(p, ((uint64_t)tag << 32) | v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint64_t ld_tag(const uint64_t *p) {
  return __hip_atomic_load(const_cast<uint64_t *>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint32_t tag_of(uint64_t v) { return (uint32_t)(v >> 32); }

// 16 bytes at base + off (base uniform over the wave), read past the work-group's caches as the agent-scope loads
// above are (the SC1 policy bit), in one request: a buffer load, whose resource is built from the uniform base.
// Records written by single 8-byte stores stay whole in it (an aligned 16-byte piece of one cache line).
__device__ __forceinline__ uint4 ld_co16(const void *base, uint32_t off) {
  typedef uint32_t v4u_t __attribute__((ext_vector_type(4)));
  constexpr int kSc1 = 16;                   // cache policy: SC1 (agent-coherent)
  constexpr uint32_t kRsrcWord3 = 0x00020000u;  // raw buffer: 32-bit data format, no swizzle
  const uint64_t b = (uint64_t)base;
  // readfirstlane returns int: each half goes through uint32_t, or the low half would sign-extend into the high.
  const uint32_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)(b >> 32));
  const uint32_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)b);
  const uint64_t bu = ((uint64_t)hi << 32) | lo;
  const __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc((void *)bu, 0, 0xffffffffu, kRsrcWord3);
  const v4u_t v = __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, kSc1);
  return make_uint4(v.x, v.y, v.z, v.w);
}

// 16 bytes to base + off (base uniform over the wave), written through to the agent's coherence point (SC1) in one
// request: the store counterpart of ld_co16.
__device__ __forceinline__ void st_co16(void *base, uint32_t off, uint4 v) {
  typedef uint32_t v4u_t __attribute__((ext_vector_type(4)));
  constexpr int kSc1 = 16;
  constexpr uint32_t kRsrcWord3 = 0x00020000u;
  const uint64_t b = (uint64_t)base;
  const uint32_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)(b >> 32));
  const uint32_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)b);
  const uint64_t bu = ((uint64_t)hi << 32) | lo;
  const __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc((void *)bu, 0, 0xffffffffu, kRsrcWord3);
  __builtin_amdgcn_raw_buffer_store_b128(v4u_t{v.x, v.y, v.z, v.w}, r, off, 0, kSc1);
}

// A word of a quantised unit: to global memory (coherent, for other work-groups of the launch) or to LDS (for this
// one), or with kPlain a plain store (read by later launches only).
template <bool kLds, typename T, bool kPlain = false>
__device__ __forceinline__ void put_word(uint8_t *out, uint32_t off, T v) {
  if constexpr (kLds || kPlain) {
    *(T *)(out + off) = v;
  } else {
    st_co((T *)(out + off), v);
  }
}

// The byte offset of codes 8 j .. 8 j + 7 of a unit in the prefill (matrix-core) order: the eight bytes lane group
// g = j % 4 takes of 32-value block b = j / 4 sit next to those it takes of block b ^ 1, so that one 16-byte read gives
// a lane its operand of a v_mfma_i32_16x16x64_i8 (blocks 2 c and 2 c + 1: 64 c + 16 g, then + 8 for the odd block).
__host__ __device__ __forceinline__ constexpr uint32_t mfma_code_off(uint32_t j) {
  return 64 * (j / 8) + 16 * (j % 4) + 8 * ((j / 4) % 2);
}

// A float through dpp_u32 (device_math.h's DPP exchanges inside a 16-lane row).
template <int kCtrl>
__device__ __forceinline__ float dpp_f32(float v) {
  return __uint_as_float(dpp_u32<kCtrl>(__float_as_uint(v)));
}

// One activation unit (256 values) quantised by a half-wave, eight values a lane (lane l32 holds values 8 l32..+7),
// with the CPU path's rules: q8_K (quantize_row_q8_K_ref) or q8_0 (the x86 quantize_row_q8_0). out is in global
// memory, or in LDS when kLds. kSplitG: q8_K's block sums as the f16 split at kActSplitH in place of the int32
// sums. kMfma: the codes in the prefill order (mfma_code_off) instead of value order. kPlain:
// plain global stores (the unit is read by later launches only). kDpp: the exchanges inside 16-lane rows as DPP
// moves (the same results: the combines are exact and order-free); all 32 lanes of the half-wave take part.
template <bool kLds = false, bool kSplitG = false, bool kMfma = false, bool kPlain = false, bool kDpp = false>
__device__ __forceinline__ void quant_unit(const float v[8], uint32_t l32, uint32_t act_type, uint8_t *out) {
  const uint32_t coff = kMfma ? mfma_code_off(l32) : 8 * l32;
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
    // The largest |v|, the first of equals: a commutative and associative combine, so any pairing order gives it.
    const auto take = [&](float oa, float om, uint32_t oi) {
      if (oa > amax || (oa == amax && oi < at)) amax = oa, mx = om, at = oi;
    };
    if constexpr (kDpp) {
      take(dpp_f32<kDppXor1>(amax), dpp_f32<kDppXor1>(mx), dpp_u32<kDppXor1>(at));
      take(dpp_f32<kDppXor2>(amax), dpp_f32<kDppXor2>(mx), dpp_u32<kDppXor2>(at));
      take(dpp_f32<kDppHalfMirror>(amax), dpp_f32<kDppHalfMirror>(mx), dpp_u32<kDppHalfMirror>(at));
      take(dpp_f32<kDppMirror>(amax), dpp_f32<kDppMirror>(mx), dpp_u32<kDppMirror>(at));
      take(__shfl_xor(amax, 16, 32), __shfl_xor(mx, 16, 32), (uint32_t)__shfl_xor((int)at, 16, 32));
    } else {
#pragma unroll
      for (int o = 16; o > 0; o >>= 1) take(__shfl_xor(amax, o, 32), __shfl_xor(mx, o, 32), (uint32_t)__shfl_xor((int)at, o, 32));
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
    if constexpr (kDpp) {
      part += (int)dpp_u32<kDppXor1>((uint32_t)part);
      part += (int)dpp_u32<kDppXor2>((uint32_t)part);
    } else {
      part += __shfl_xor(part, 1, 32);
      part += __shfl_xor(part, 2, 32);
    }
    put_word<kLds, uint64_t, kPlain>(out, coff, ((uint64_t)code[1] << 32) | code[0]);
    if constexpr (kSplitG) {
      // Block sum j = l32 / 4 split as 64 hi + lo (hi in [-64, 63], lo in [0, 63]), both as f16, at kActSplitH.
      if ((l32 & 3u) == 0) {
        const int lo = part & 63;
        put_word<kLds, uint16_t, kPlain>(out, kActSplitH + l32 / 2, f2h((float)lo));
        put_word<kLds, uint16_t, kPlain>(out, kActSplitH + 16 + l32 / 2, f2h((float)(part - lo)));
      }
    } else {
      if ((l32 & 3u) == 0) put_word<kLds, int, kPlain>(out, kActSums + l32, part);
    }
    if (l32 == 0) put_word<kLds, float, kPlain>(out, kActScales, d);
  } else {  // q8_0: blocks of 32, four lanes each
    float amax = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; i++) amax = fmaxf(amax, fabsf(v[i]));
    if constexpr (kDpp) {
      amax = fmaxf(amax, dpp_f32<kDppXor1>(amax));
      amax = fmaxf(amax, dpp_f32<kDppXor2>(amax));
    } else {
      amax = fmaxf(amax, __shfl_xor(amax, 1, 32));
      amax = fmaxf(amax, __shfl_xor(amax, 2, 32));
    }
    const float d = __fdiv_rn(amax, 127.0f), id = amax != 0.0f ? __fdiv_rn(127.0f, amax) : 0.0f;
#pragma unroll
    for (int i = 0; i < 8; i++) {
      const int q = nearest_int(__fmul_rn(v[i], id));
      code[i / 4] |= ((uint32_t)q & 0xffu) << (8 * (i % 4));
    }
    put_word<kLds, uint64_t, kPlain>(out, coff, ((uint64_t)code[1] << 32) | code[0]);
    if ((l32 & 3u) == 0) put_word<kLds, float, kPlain>(out, kActScales + l32, h2f(f2h(d)));
    if ((l32 & 3u) == 0) put_word<kLds, int, kPlain>(out, kActSums + l32, 0);
  }
}

}  // namespace c0ven
