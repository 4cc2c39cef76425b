// Device-side scalar arithmetic with the bits the CPU path gives: libm's expf, IEEE conversions, ggml's rounding.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace c0ven {

// 2^(i/32) for i = 0..31, each the nearest double, as its bits minus i << 47 (so that adding k << 47 for k = 32 q + i
// gives 2^(k/32) once the exponent carries in q). tests/test_device_tables.py recomputes them exactly.
#define C0VEN_EXP2_TAB_VALUES \
    0x3ff0000000000000ull, 0x3fefd9b0d3158574ull, 0x3fefb5586cf9890full, 0x3fef9301d0125b51ull, \
    0x3fef72b83c7d517bull, 0x3fef54873168b9aaull, 0x3fef387a6e756238ull, 0x3fef1e9df51fdee1ull, \
    0x3fef06fe0a31b715ull, 0x3feef1a7373aa9cbull, 0x3feedea64c123422ull, 0x3feece086061892dull, \
    0x3feebfdad5362a27ull, 0x3feeb42b569d4f82ull, 0x3feeab07dd485429ull, 0x3feea47eb03a5585ull, \
    0x3feea09e667f3bcdull, 0x3fee9f75e8ec5f74ull, 0x3feea11473eb0187ull, 0x3feea589994cce13ull, \
    0x3feeace5422aa0dbull, 0x3feeb737b0cdc5e5ull, 0x3feec49182a3f090ull, 0x3feed503b23e255dull, \
    0x3feee89f995ad3adull, 0x3feeff76f2fb5e47ull, 0x3fef199bdd85529cull, 0x3fef3720dcef9069ull, \
    0x3fef5818dcfba487ull, 0x3fef7c97337b9b5full, 0x3fefa4afa2a490daull, 0x3fefd0765b6e4540ull
__device__ __constant__ static const uint64_t kExp2Tab[32] = {C0VEN_EXP2_TAB_VALUES};

// expf with the bits of glibc 2.35's x86-64 expf on a CPU with FMA (its __expf_fma, which the host's libm runs and
// which the CPU path's std::exp calls). The method is ARM optimized-routines' expf (MIT/Apache-2.0; glibc
// sysdeps/ieee754/flt-32/e_expf.c): x / ln2 * 32 = k + r with |r| <= 1/2, 2^(k/32) from the table, 2^(r/32) from a
// cubic, all in double, rounded once to float. The fused multiply-adds are where the FMA build fuses; everything else
// is a single IEEE operation (the library builds with -ffp-contract=off). tab is the table above (in constant or LDS
// memory on the device, a host copy on the CPU): the same source runs on both, and tests/test_expf.py checks the host
// build against libm's expf on all 2^32 inputs.
__host__ __device__ __forceinline__ float expf_libm(float x, const uint64_t *tab) {
  // The main path runs for every input and the out-of-range cases are selected at the end, so the code has no
  // branches: a wave evaluates several of these interleaved. Outside (-0x1.9fe368p6, 0x1.62e42ep6) the result is
  // 0 or infinity (both infinities included), a NaN gives x + x; those are exactly libm's special cases.
  const double InvLn2N = 0x1.71547652b82fep+0 * 32, Shift = 0x1.8p+52;
  const double C0 = 0x1.c6af84b912394p-5 / 32 / 32 / 32, C1 = 0x1.ebfce50fac4f3p-3 / 32 / 32,
               C2 = 0x1.62e42ff0c52d6p-1 / 32;
  const bool under = x < -0x1.9fe368p6f, over = x > 0x1.62e42ep6f, nan = x != x;
  const double xd = (double)((under | over | nan) ? 0.0f : x);
  double kd = __builtin_fma(InvLn2N, xd, Shift);
  const uint64_t ki = __builtin_bit_cast(uint64_t, kd);
  kd = kd - Shift;
  const double r = __builtin_fma(InvLn2N, xd, -kd);
  const uint64_t t = tab[ki % 32] + (ki << 47);
  const double sc = __builtin_bit_cast(double, t);
  const double z = __builtin_fma(C0, r, C1);
  const double r2 = r * r;
  double y = __builtin_fma(C2, r, 1.0);
  y = __builtin_fma(z, r2, y);
  y = y * sc;
  float res = (float)y;
  res = under ? 0.0f : res;
  res = over ? __builtin_bit_cast(float, 0x7f800000u) : res;
  return nan ? x + x : res;
}

// silu(g) * u with the optional clamp, each step rounded as the CPU path's g / (1 + expf(-g)) * u.
__host__ __device__ __forceinline__ float swiglu_one(float g, float u, float limit, const uint64_t *tab) {
  if (limit > 0.0f) {
    g = g < limit ? g : limit;
    u = u < -limit ? -limit : (u > limit ? limit : u);
  }
  const float den = 1.0f + expf_libm(-g, tab);
  return (g / den) * u;
}

__host__ __device__ __forceinline__ float sigmoid_libm(float z, const uint64_t *tab) {
  return 1.0f / (1.0f + expf_libm(-z, tab));
}

__device__ __forceinline__ float h2f(uint16_t h) { return (float)__builtin_bit_cast(_Float16, h); }
__device__ __forceinline__ uint16_t f2h(float f) { return __builtin_bit_cast(uint16_t, (_Float16)f); }
__device__ __forceinline__ float bf2f(uint16_t b) { return __uint_as_float((uint32_t)b << 16); }
// bf16 by round to nearest even (ggml's GGML_FP32_TO_BF16), NaN kept quiet.
__device__ __forceinline__ float round_bf16(float f) {
  // gfx950's v_cvt_pk_bf16_f32 rounds to nearest even and quiets a NaN exactly this way: checked on the GPU against
  // the bit formula (x + 0x7fff + lsb, truncated; NaN: truncated with the quiet bit set) for all 2^32 inputs.
  return __uint_as_float((uint32_t)__builtin_bit_cast(unsigned short, (__bf16)f) << 16);
}
// Two at once (one v_cvt_pk_bf16_f32).
__device__ __forceinline__ void round_bf16_2(float a, float b, float &ra, float &rb) {
  typedef float f2 __attribute__((ext_vector_type(2)));
  typedef __bf16 b2 __attribute__((ext_vector_type(2)));
  const uint32_t w = __builtin_bit_cast(uint32_t, __builtin_convertvector(f2{a, b}, b2));
  ra = __uint_as_float(w << 16), rb = __uint_as_float(w & 0xffff0000u);
}

// ggml's nearest_int: round half to even, |v| < 2^22.
__device__ __forceinline__ int nearest_int(float v) { return (int)__builtin_rintf(v); }

__device__ __forceinline__ int dot4(uint32_t a, uint32_t b, int c) {
  return __builtin_amdgcn_sdot4((int)a, (int)b, c, false);
}

// Wave64 reductions (all lanes get the result).
__device__ __forceinline__ float wave_max(float v) {
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}
__device__ __forceinline__ int wave_sum_i(int v) {
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}
__device__ __forceinline__ double wave_sum_d(double v) {
  for (int o = 32; o > 0; o >>= 1) v = __dadd_rn(v, __shfl_xor(v, o, 64));
  return v;
}

// DPP lane exchanges (gfx9 controls): quad_perm(1,0,3,2) = lane ^ 1, quad_perm(2,3,0,1) = lane ^ 2,
// quad_perm(3,2,1,0) = 3 - lane within 4, row_half_mirror = 7 - lane within 8, row_mirror = 15 - lane within 16. Each pairs a lane with one in the other half
// of its 2, 4, 8 or 16, so four steps reduce a row of 16 with every lane holding the result.
template <int kCtrl>
__device__ __forceinline__ uint32_t dpp_u32(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, kCtrl, 0xf, 0xf, false);
}
constexpr int kDppXor1 = 0xB1, kDppXor2 = 0x4E, kDppQuadRev = 0x1B, kDppHalfMirror = 0x141, kDppMirror = 0x140;
constexpr int kDppShr1 = 0x111;  // row_shr:1 (lane - 1 within a row of 16)

__device__ __forceinline__ uint32_t readlane_u32(uint32_t v, int l) { return (uint32_t)__builtin_amdgcn_readlane((int)v, l); }

// The wave's largest / smallest u32, wave-uniform.
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
  v = max(v, dpp_u32<kDppXor1>(v));
  v = max(v, dpp_u32<kDppXor2>(v));
  v = max(v, dpp_u32<kDppHalfMirror>(v));
  v = max(v, dpp_u32<kDppMirror>(v));
  return max(max(readlane_u32(v, 0), readlane_u32(v, 16)), max(readlane_u32(v, 32), readlane_u32(v, 48)));
}
__device__ __forceinline__ uint32_t wave_min_u32(uint32_t v) {
  v = min(v, dpp_u32<kDppXor1>(v));
  v = min(v, dpp_u32<kDppXor2>(v));
  v = min(v, dpp_u32<kDppHalfMirror>(v));
  v = min(v, dpp_u32<kDppMirror>(v));
  return min(min(readlane_u32(v, 0), readlane_u32(v, 16)), min(readlane_u32(v, 32), readlane_u32(v, 48)));
}

template <int kCtrl>
__device__ __forceinline__ double dpp_f64(double v) {
  const uint64_t b = __builtin_bit_cast(uint64_t, v);
  const uint64_t r = (uint64_t)dpp_u32<kCtrl>((uint32_t)b) | ((uint64_t)dpp_u32<kCtrl>((uint32_t)(b >> 32)) << 32);
  return __builtin_bit_cast(double, r);
}
__device__ __forceinline__ double readlane_f64(double v, int l) {
  const uint64_t b = __builtin_bit_cast(uint64_t, v);
  return __builtin_bit_cast(double, (uint64_t)readlane_u32((uint32_t)b, l) | ((uint64_t)readlane_u32((uint32_t)(b >> 32), l) << 32));
}
// The wave's fp64 sum in one fixed order (butterflies within rows of 16, then the four rows pairwise), wave-uniform.
__device__ __forceinline__ double wave_sum_f64(double v) {
  v = __dadd_rn(v, dpp_f64<kDppXor1>(v));
  v = __dadd_rn(v, dpp_f64<kDppXor2>(v));
  v = __dadd_rn(v, dpp_f64<kDppHalfMirror>(v));
  v = __dadd_rn(v, dpp_f64<kDppMirror>(v));
  return __dadd_rn(__dadd_rn(readlane_f64(v, 0), readlane_f64(v, 16)), __dadd_rn(readlane_f64(v, 32), readlane_f64(v, 48)));
}
// A float's bits as a u32 that orders as the floats do (-0 taken as +0), and back.
__device__ __forceinline__ uint32_t float_key(float f) {
  uint32_t u = __float_as_uint(__fadd_rn(f, 0.0f));
  return u ^ ((u >> 31) ? 0xffffffffu : 0x80000000u);
}
__device__ __forceinline__ float key_float(uint32_t k) { return __uint_as_float((k & 0x80000000u) ? (k ^ 0x80000000u) : ~k); }

}  // namespace c0ven
