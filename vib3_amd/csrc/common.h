// common.h — device helpers shared by the gfx950 kernels of libvib3_hip.
//
// Wave64 everywhere: reductions use DPP within 16-lane rows plus v_readlane across rows.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/vib3_hip.h"

namespace vib3 {

typedef _Float16 half_t;
typedef _Float16 h2 __attribute__((ext_vector_type(2)));

constexpr int kWave = 64;

// ------------------------------------------------------------------------- conversions

__device__ __forceinline__ float bf16_to_f32(uint16_t b) { return __uint_as_float((uint32_t)b << 16); }

__device__ __forceinline__ float f16_to_f32(uint16_t b) {
  return (float)__builtin_bit_cast(half_t, b);
}

__device__ __forceinline__ uint16_t f32_to_f16_bits(float f) {
  return __builtin_bit_cast(uint16_t, (half_t)f);  // v_cvt_f16_f32, round to nearest even
}

// f32 -> bf16 bits, round to nearest even, NaN kept quiet (same rule as the `half` crate).
__device__ __forceinline__ uint16_t f32_to_bf16_bits(float f) {
  uint32_t x = __float_as_uint(f);
  if ((x & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((x >> 16) | 0x40u);
  uint32_t lsb = (x >> 16) & 1u;
  return (uint16_t)((x + 0x7fffu + lsb) >> 16);
}

// Load element i of an activation vector of dtype dt as f32.
__device__ __forceinline__ float load_act(const void* p, int dt, size_t i) {
  if (dt == VIB3_DT_F32) return ((const float*)p)[i];
  uint16_t b = ((const uint16_t*)p)[i];
  return dt == VIB3_DT_F16 ? f16_to_f32(b) : bf16_to_f32(b);
}

// INT4 group scale: bf16 or f16 bits; not finite or not > 0 -> 1/8 (kernels.rs:2791-2797).
__device__ __forceinline__ float decode_scale(uint16_t bits, int sdt) {
  float s = sdt == VIB3_DT_F16 ? f16_to_f32(bits) : bf16_to_f32(bits);
  return (s > 0.0f && s < __builtin_huge_valf()) ? s : 0.125f;
}

// ------------------------------------------------------------------------- wave reductions

template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xf, 0xf, true));
}

// Sum over the 64 lanes; the result is wave-uniform.
__device__ __forceinline__ float wave_sum(float v) {
  v += dpp<0xB1>(v);   // quad_perm [1,0,3,2]
  v += dpp<0x4E>(v);   // quad_perm [2,3,0,1]
  v += dpp<0x141>(v);  // row_half_mirror
  v += dpp<0x140>(v);  // row_mirror: every lane holds its 16-lane row sum
  float r0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
  float r1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16));
  float r2 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
  float r3 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48));
  return (r0 + r1) + (r2 + r3);
}

// o + w * d with the product rounded before the add (never fused into an FMA), the way the
// reference's `*o += weight * x` compiles.
__device__ __forceinline__ float add_mul_rn(float o, float w, float d) {
#pragma clang fp contract(off)
  return o + w * d;
}

__device__ __forceinline__ int lane_id() { return (int)(threadIdx.x & (kWave - 1)); }

// Wait for this wave's LDS (and scalar memory) operations only: s_waitcnt lgkmcnt(0) with the
// vector-memory and export counters left at their maximum, so loads still in flight (streamed
// weights issued ahead of time) are not drained.
__device__ __forceinline__ void wait_lgkm() { __builtin_amdgcn_s_waitcnt(0xC07F); }

// ------------------------------------------------------------------------- INT4 chunk dot
//
// A chunk is 16 bytes of one weight row = 32 consecutive columns. Word i of the chunk holds
// columns 8i..8i+7 as nibbles [c0 c1 | c2 c3 | c4 c5 | c6 c7] (low nibble first per byte).
// Masking a word with 0x000F000F leaves (c0, c4) as the two halves of a packed f16 pair whose
// bit patterns are the raw codes q, i.e. the f16 subnormals q * 2^-24; 0x00F000F0 leaves
// (c1, c5) as 16q * 2^-24; the same on word >> 8 gives (c2, c6) and (c3, c7). One v_dot2 per
// pair against the matching activation pair accumulates q * x exactly (products of an 4-bit
// and an 11-bit significand) into f32. The -8 offset is applied once per chunk through the
// precomputed sum of the chunk's activations, and 2^24 is folded into the final row scale.

struct XChunk {
  h2 a[4], b[4], c[4], d[4];  // (x0,x4) (x1,x5) (x2,x6) (x3,x7) of each word
  float xs8;                   // 8 * 2^-24 * sum of the chunk's activations
};

struct XWords {  // an XChunk as its 17 words (xs8 last)
  uint32_t w[17];
};
static_assert(sizeof(XWords) == sizeof(XChunk), "XChunk is 17 words");

__device__ __forceinline__ h2 as_h2(uint32_t v) { return __builtin_bit_cast(h2, v); }

__device__ __forceinline__ float chunk_dot(const uint4 w, const XChunk& x) {
  const uint32_t v[4] = {w.x, w.y, w.z, w.w};
  float c1 = 0.0f, c2 = 0.0f;
#pragma unroll
  for (int i = 0; i < 4; i++) {
    const uint32_t u = v[i], t = v[i] >> 8;
    c1 = __builtin_amdgcn_fdot2(as_h2(u & 0x000F000Fu), x.a[i], c1, false);
    c2 = __builtin_amdgcn_fdot2(as_h2(u & 0x00F000F0u), x.b[i], c2, false);
    c1 = __builtin_amdgcn_fdot2(as_h2(t & 0x000F000Fu), x.c[i], c1, false);
    c2 = __builtin_amdgcn_fdot2(as_h2(t & 0x00F000F0u), x.d[i], c2, false);
  }
  return __builtin_fmaf(c2, 0.0625f, c1) - x.xs8;
}

constexpr float kTwo24 = 16777216.0f;
constexpr float kTwoM24 = 5.9604644775390625e-08f;
constexpr float kF16Normal = 6.103515625e-05f;

// Fill hi (and lo, the f16 residual) for chunk c from 32 f32 activations; returns whether the
// residual is needed (some |x| in the f16 normal range is not exactly representable).
__device__ __forceinline__ bool make_chunk(const float* xv, XChunk& hi, XChunk& lo) {
  bool need = false;
  float sum = 0.0f;
#pragma unroll
  for (int i = 0; i < 4; i++) {
    float x[8];
#pragma unroll
    for (int j = 0; j < 8; j++) x[j] = xv[8 * i + j];
    half_t h[8], l[8];
#pragma unroll
    for (int j = 0; j < 8; j++) {
      h[j] = (half_t)x[j];
      float r = x[j] - (float)h[j];
      l[j] = (half_t)r;
      need |= (r != 0.0f) && (__builtin_fabsf(x[j]) >= kF16Normal);
      sum += x[j];
    }
    hi.a[i] = h2{h[0], h[4]};
    hi.b[i] = h2{h[1], h[5]};
    hi.c[i] = h2{h[2], h[6]};
    hi.d[i] = h2{h[3], h[7]};
    lo.a[i] = h2{l[0], l[4]};
    lo.b[i] = h2{l[1], l[5]};
    lo.c[i] = h2{l[2], l[6]};
    lo.d[i] = h2{l[3], l[7]};
  }
  hi.xs8 = 8.0f * kTwoM24 * sum;
  lo.xs8 = 0.0f;
  return need;
}

// Activation modes of the INT4 row kernels: f16 pairs (exact for f16 / bf16 activations),
// f32 split into hi + lo f16 pairs (two dot products per pair), or f32 as int16 block fixed
// point per 32-element chunk (one integer dot product per pair); kXi16n: kXi16 of RMSNorm(x),
// the norm fused into the kernel (x the f32 residual stream).
enum { kXf16 = 0, kXsplit = 1, kXi16 = 2, kXi16n = 3 };

// Chunk of 32 f32 activations as int16 pairs x_i = rint(x * 2^sh), sh = 15 - E with E the
// exponent of the chunk's largest |x| (|x_i| <= 32767), in the slots of hi (the pair layout
// of chunk_dot); hi.xs8 = the bits of 8 * sum(x_i) as an int, lo.xs8 = 2^(-sh-24), the factor
// that brings the integer dot back to chunk_dot's 2^-24 units. Error per element at most half
// a unit of 2^-sh: 2^-16 of the chunk's largest value.
__device__ __forceinline__ void make_chunk_i16(const float* xv, XChunk& hi, XChunk& lo) {
  float amax = 0.0f;
#pragma unroll
  for (int j = 0; j < 32; j++) amax = fmaxf(amax, __builtin_fabsf(xv[j]));
  int E = 0;
  (void)__builtin_frexpf(amax, &E);  // amax = f 2^E, f in [0.5, 1)
  const int sh = amax > 0.0f ? 15 - E : 0;
  int sum = 0;
#pragma unroll
  for (int i = 0; i < 4; i++) {
    int q[8];
#pragma unroll
    for (int j = 0; j < 8; j++) {
      const float t = __builtin_rintf(__builtin_ldexpf(xv[8 * i + j], sh));
      q[j] = (int)fminf(fmaxf(t, -32767.0f), 32767.0f);
      sum += q[j];
    }
    auto pk = [](int a, int b) { return as_h2(((uint32_t)a & 0xffffu) | ((uint32_t)b << 16)); };
    hi.a[i] = pk(q[0], q[4]);
    hi.b[i] = pk(q[1], q[5]);
    hi.c[i] = pk(q[2], q[6]);
    hi.d[i] = pk(q[3], q[7]);
  }
  hi.xs8 = __int_as_float(8 * sum);
  lo.xs8 = __builtin_ldexpf(1.0f, -sh - 24);
}

typedef short s2 __attribute__((ext_vector_type(2)));

// chunk_dot for an int16 chunk: sum (q - 8) x_i exactly in integers, times 2^(-sh-24).
__device__ __forceinline__ float chunk_dot_i16(const uint4 w, const XChunk& x, float mult) {
  const uint32_t v[4] = {w.x, w.y, w.z, w.w};
  int c1 = 0, c2 = 0;
#pragma unroll
  for (int i = 0; i < 4; i++) {
    const uint32_t u = v[i], t = v[i] >> 8;
    c1 = __builtin_amdgcn_sdot2(__builtin_bit_cast(s2, u & 0x000F000Fu), __builtin_bit_cast(s2, x.a[i]), c1, false);
    c2 = __builtin_amdgcn_sdot2(__builtin_bit_cast(s2, u & 0x00F000F0u), __builtin_bit_cast(s2, x.b[i]), c2, false);
    c1 = __builtin_amdgcn_sdot2(__builtin_bit_cast(s2, t & 0x000F000Fu), __builtin_bit_cast(s2, x.c[i]), c1, false);
    c2 = __builtin_amdgcn_sdot2(__builtin_bit_cast(s2, t & 0x00F000F0u), __builtin_bit_cast(s2, x.d[i]), c2, false);
  }
  return (float)(c1 + (c2 >> 4) - __float_as_int(x.xs8)) * mult;
}

__device__ __forceinline__ void zero_chunk(XChunk& c) {
#pragma unroll
  for (int i = 0; i < 4; i++) c.a[i] = c.b[i] = c.c[i] = c.d[i] = h2{(half_t)0, (half_t)0};
  c.xs8 = 0.0f;
}

// Load the 32 activations of chunk c (columns 32c..32c+31) as f32.
__device__ __forceinline__ void load_chunk_act(const void* x, int dt, int c, float* out) {
  if (dt == VIB3_DT_F32) {
    const float4* p = (const float4*)((const float*)x + 32 * (size_t)c);
#pragma unroll
    for (int i = 0; i < 8; i++) {
      float4 v = p[i];
      out[4 * i] = v.x; out[4 * i + 1] = v.y; out[4 * i + 2] = v.z; out[4 * i + 3] = v.w;
    }
  } else {
    const uint4* p = (const uint4*)((const uint16_t*)x + 32 * (size_t)c);
#pragma unroll
    for (int i = 0; i < 4; i++) {
      uint4 v = p[i];
      uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
      for (int j = 0; j < 4; j++) {
        uint16_t b0 = (uint16_t)(w[j] & 0xffff), b1 = (uint16_t)(w[j] >> 16);
        out[8 * i + 2 * j] = dt == VIB3_DT_F16 ? f16_to_f32(b0) : bf16_to_f32(b0);
        out[8 * i + 2 * j + 1] = dt == VIB3_DT_F16 ? f16_to_f32(b1) : bf16_to_f32(b1);
      }
    }
  }
}

// Non-temporal 16-byte load of streamed weights (read once per token).
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

typedef __attribute__((address_space(1))) const u32x4 global_u32x4;

__device__ __forceinline__ uint4 ld_stream(const uint8_t* p) {
  const u32x4 v = __builtin_nontemporal_load((global_u32x4*)p);
  return make_uint4(v.x, v.y, v.z, v.w);
}

// 2-byte load through the global address space (pointers read from page tables are generic;
// a flat load would also count against the LDS counter and force conservative waits).
__device__ __forceinline__ uint16_t ld_u16(const uint16_t* p) {
  return *(__attribute__((address_space(1))) const uint16_t*)p;
}

// Page-table entry through the constant address space: with a wave-uniform address this is a
// scalar load (s_load), so waiting for it never involves the vector memory counter. Page tables
// are read-only while a kernel runs.
__device__ __forceinline__ uint64_t ld_table(const uint64_t* p) {
  return *(const __attribute__((address_space(4))) uint64_t*)p;
}

// A pointer every lane holds the same value of (e.g. read from LDS), moved to SGPRs so that
// loads through it are scalar and their waits do not involve the vector memory counter.
template <typename T>
__device__ __forceinline__ T* uniform_ptr(T* p) {
  const uint64_t v = (uint64_t)(uintptr_t)p;
  const uint32_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)v);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(v >> 32));
  return (T*)(uintptr_t)(((uint64_t)hi << 32) | lo);
}

// ------------------------------------------------------------------------- matrix addressing
//
// An INT4 matrix is either flat (data rows then scale rows at explicit pointers) or a list of
// pages from a page table, each page [rows x pk][rows x ng x 2] with rows_per_page rows
// (the last page may be short). row() resolves one row with a single table read.

struct MatRef {
  const uint64_t* table;  // paged: table[page] = page address
  const uint8_t* data;    // flat: data rows
  const uint16_t* scales; // flat: scale rows
  int rpp;                // rows per page (paged)
  int rows;               // rows of the whole matrix
  uint64_t magic;         // ceil(2^32 / rpp): page = (row * magic) >> 32 (exact for rows < 2^16)
};

__host__ __device__ inline uint64_t page_magic(int rpp) {
  return ((1ull << 32) + (uint64_t)rpp - 1) / (uint64_t)rpp;
}

// Row r of a matrix: data and scale-row pointers. Paged: one table read, no branch, no divide.
template <bool PAGED>
__device__ __forceinline__ void mat_row(const MatRef& m, int r, int pk, int ng, const uint8_t*& d,
                                        const uint16_t*& s) {
  if (PAGED) {
    const int p = (int)(((uint64_t)(uint32_t)r * m.magic) >> 32);
    const int rr = r - p * m.rpp;
    const int rows_here = min(m.rpp, m.rows - p * m.rpp);
    const uint8_t* base = (const uint8_t*)ld_table(m.table + p);
    d = base + (size_t)rr * pk;
    s = (const uint16_t*)(base + (size_t)rows_here * pk) + (size_t)rr * ng;
  } else {
    d = m.data + (size_t)r * pk;
    s = m.scales + (size_t)r * ng;
  }
}

}  // namespace vib3

// s_waitcnt for at most n vector-memory operations outstanding (n < 64; lgkm and exp counts
// left at their maximum)
#define VIB3_WAIT_VM(n) __builtin_amdgcn_s_waitcnt(0x0F70 | ((n) & 15) | (((n) >> 4) << 14))

// Timeline probes for kernel-internal phases: compiled in only when VIB3_TRACE is defined (a
// profiling build; the buffer pointer is set per translation unit by vib3_trace_set in
// int4_gemv.hip); each probe stores the 100 MHz real-time counter for (workgroup, point).
#ifdef VIB3_TRACE
static __device__ uint64_t* vib3_trace_buf;
#define VIB3_TRACE_POINT(k)                                                          \
  do {                                                                               \
    if (threadIdx.x == 0) vib3_trace_buf[blockIdx.x * 16 + (k)] = __builtin_amdgcn_s_memrealtime(); \
  } while (0)
#define VIB3_TRACE_VALUE(k, v)                                                       \
  do {                                                                               \
    if (threadIdx.x == 0) vib3_trace_buf[blockIdx.x * 16 + (k)] = (uint64_t)(v);       \
  } while (0)
#else
#define VIB3_TRACE_VALUE(k, v) \
  do {                         \
  } while (0)
#define VIB3_TRACE_POINT(k) \
  do {                      \
  } while (0)
#endif

// Launch-error plumbing shared by the launchers.
#define VIB3_RETURN_LAUNCH()                      \
  do {                                            \
    hipError_t _e = hipGetLastError();            \
    return _e == hipSuccess ? 0 : (int)_e;        \
  } while (0)
