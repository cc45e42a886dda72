// fp4.h — device pieces of the block-scaled FP4 (E2M1 x E8M0) arithmetic shared by the fused
// NVFP4 MoE (fp4_fused.hip) and the per-page NVFP4 launchers (fp4_pages.hip): the E8M0 and
// E2M1 rounding rules of the reference's quantizers, an exp whose every operation the oracle
// repeats, exact group dot products on decoded pairs, and f64 lane shuffles.
#pragma once

#include "common.h"

namespace vib3 {
namespace {

typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));

constexpr int kFp4MaxActive = 8;  // MOE_MAX_EXPERTS (kernels.cu:5331)
#ifndef VIB3_FP4_DEPTH
#define VIB3_FP4_DEPTH 2  // 1 KB tile pairs in flight per matrix stream (build-time knob)
#endif
constexpr int kFp4Depth = VIB3_FP4_DEPTH;

// ------------------------------------------------------------------------- scalar pieces

// E8M0 exponent of a group's scale from its absolute maximum (kernels.cu:2759-2768):
// round(log2(amax)) - 2 + 127 clamped to [0, 254], with round(log2) taken exactly as
// floor(log2) + (mantissa > sqrt 2) (the float just below sqrt 2 has mantissa 0x3504f3).
__device__ __forceinline__ uint32_t e8m0_of_amax(float amax) {
  if (!(amax > 0.0f)) return 0;
  const uint32_t b = __float_as_uint(amax);
  const int E = (int)(b >> 23);
  if (E == 0) return 0;  // subnormal: log2 < -126, below the clamp
  const int n = E - 127 + ((b & 0x7fffff) > 0x3504f3 ? 1 : 0);
  const int biased = n + 125;
  return (uint32_t)(biased < 0 ? 0 : biased > 254 ? 254 : biased);
}

// Round-to-nearest-even onto the E2M1 grid {0, .5, 1, 1.5, 2, 3, 4, 6}, saturating at 6,
// sign kept (cvt.rn.satfinite semantics of __nv_fp4x4_e2m1, used at kernels.cu:3227).
__device__ __forceinline__ uint32_t e2m1_rne(float v) {
  const uint32_t sign = (__float_as_uint(v) >> 31) << 3;
  const float a = fabsf(v);
  uint32_t c;
  if (a <= 0.25f) c = 0;
  else if (a < 0.75f) c = 1;
  else if (a <= 1.25f) c = 2;
  else if (a < 1.75f) c = 3;
  else if (a <= 2.5f) c = 4;
  else if (a < 3.5f) c = 5;
  else if (a <= 5.0f) c = 6;
  else c = 7;
  return sign | c;
}

// 1 / 2^(e - 127), the exact reciprocal of an E8M0 scale (e = 0 reads as 0 there, whose
// reciprocal is +inf, kernels.cu:2770-2777 with __frcp_rn).
__device__ __forceinline__ float e8m0_inv(uint32_t e) {
  return e == 0 ? __builtin_huge_valf() : __uint_as_float((254u - e) << 23);
}

// e^x by Cody-Waite reduction x = n ln2 + r (ln2 split in a 15-bit head and a tail, so n * head
// is exact) and the degree-7 Taylor polynomial of e^r on |r| <= ln2 / 2 in Horner form, then
// ldexp. Every operation is a single IEEE rounding (no contraction), so the oracle's C version
// gives the same bits; within 2 ulp of the correctly rounded exp (tested against libm).
__device__ __forceinline__ float exp_cw(float x) {
#pragma clang fp contract(off)
  if (x != x) return x;
  if (x > 88.72283935546875f) return __builtin_huge_valf();
  if (x < -103.97208404541015625f) return 0.0f;
  const float n = __builtin_rintf(x * 1.44269502162933349609375f);
  float r = x - n * 0.693145751953125f;
  r = r - n * 1.428606765330187045e-06f;
  float p = 1.0f / 5040.0f;
  p = p * r + 1.0f / 720.0f;
  p = p * r + 1.0f / 120.0f;
  p = p * r + 1.0f / 24.0f;
  p = p * r + 1.0f / 6.0f;
  p = p * r + 0.5f;
  p = p * r + 1.0f;
  p = p * r + 1.0f;
  return __builtin_ldexpf(p, (int)n);
}

// h = (g * sigmoid(g)) * u, sigmoid(g) = 1 / (1 + e^-g), in the reference's order
// (kernels.cu:5485-5487).
__device__ __forceinline__ float swiglu_fp4(float g, float u) {
#pragma clang fp contract(off)
  const float sig = 1.0f / (1.0f + exp_cw(-g));
  return (g * sig) * u;
}

// 2^(e) as a double for e in [-254, 254] (always a normal double: exact).
__device__ __forceinline__ double pow2d(int e) {
  return __longlong_as_double((long long)(e + 1023) << 52);
}

// Sixteen split-half bytes (one group) as sixteen f16 pairs (value j, value j + 16), exact.
__device__ __forceinline__ void decode_group(const uint4 w, f16x2 (&o)[16]) {
  const uint32_t wd[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
  for (int i = 0; i < 4; i++) {
    o[4 * i + 0] = __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(wd[i], 1.0f, 0);
    o[4 * i + 1] = __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(wd[i], 1.0f, 1);
    o[4 * i + 2] = __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(wd[i], 1.0f, 2);
    o[4 * i + 3] = __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(wd[i], 1.0f, 3);
  }
}

// Exact group dot product of weight bytes `w` with a decoded activation group in LDS.
__device__ __forceinline__ float group_dot(const uint4 w, const uint4* act) {
  const uint4 a4[4] = {act[0], act[1], act[2], act[3]};
  const uint32_t aw[16] = {a4[0].x, a4[0].y, a4[0].z, a4[0].w, a4[1].x, a4[1].y, a4[1].z, a4[1].w,
                           a4[2].x, a4[2].y, a4[2].z, a4[2].w, a4[3].x, a4[3].y, a4[3].z, a4[3].w};
  f16x2 wp[16];
  decode_group(w, wp);
  float s = 0.0f;
#pragma unroll
  for (int j = 0; j < 16; j++)
    s = __builtin_amdgcn_fdot2(wp[j], __builtin_bit_cast(f16x2, aw[j]), s, false);
  return s;
}

__device__ __forceinline__ double shfl_xor_d(double v, int m) {
  const long long b = __double_as_longlong(v);
  const int lo = __shfl_xor((int)(uint32_t)b, m), hi = __shfl_xor((int)(uint32_t)(b >> 32), m);
  return __longlong_as_double(((long long)hi << 32) | (uint32_t)lo);
}

}  // namespace
}  // namespace vib3
