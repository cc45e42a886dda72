// router_dot.h — one router logit computed by a 256-thread workgroup (shared by the router
// kernel and the fused gate/up kernel, which computes the logits in its own prologue).
#pragma once

#include "common.h"
#include "kernels.h"
#include "norm.h"

namespace vib3 {

__device__ __forceinline__ void load8_act(const void* p, int dt, size_t i, float* o) {
  if (dt == VIB3_DT_F32) {
    const float4* q = (const float4*)((const float*)p + i);
    float4 a = q[0], b = q[1];
    o[0] = a.x; o[1] = a.y; o[2] = a.z; o[3] = a.w;
    o[4] = b.x; o[5] = b.y; o[6] = b.z; o[7] = b.w;
  } else {
    uint4 v = *(const uint4*)((const uint16_t*)p + i);
    uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int j = 0; j < 4; j++) {
      uint16_t lo = (uint16_t)(w[j] & 0xffff), hi = (uint16_t)(w[j] >> 16);
      o[2 * j] = dt == VIB3_DT_F16 ? f16_to_f32(lo) : bf16_to_f32(lo);
      o[2 * j + 1] = dt == VIB3_DT_F16 ? f16_to_f32(hi) : bf16_to_f32(hi);
    }
  }
}

__device__ __forceinline__ void load8_stream(const void* p, int dt, size_t i, float* o) {
  if (dt == VIB3_DT_F32) {
    const float* q = (const float*)p + i;
    uint4 a = ld_stream((const uint8_t*)q);
    uint4 b = ld_stream((const uint8_t*)(q + 4));
    o[0] = __uint_as_float(a.x); o[1] = __uint_as_float(a.y);
    o[2] = __uint_as_float(a.z); o[3] = __uint_as_float(a.w);
    o[4] = __uint_as_float(b.x); o[5] = __uint_as_float(b.y);
    o[6] = __uint_as_float(b.z); o[7] = __uint_as_float(b.w);
  } else {
    uint4 v = ld_stream((const uint8_t*)((const uint16_t*)p + i));
    uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int j = 0; j < 4; j++) {
      uint16_t lo = (uint16_t)(w[j] & 0xffff), hi = (uint16_t)(w[j] >> 16);
      o[2 * j] = dt == VIB3_DT_F16 ? f16_to_f32(lo) : bf16_to_f32(lo);
      o[2 * j + 1] = dt == VIB3_DT_F16 ? f16_to_f32(hi) : bf16_to_f32(hi);
    }
  }
}

// Dot product of x with router row e, computed by the whole 256-thread workgroup; the result is
// valid in every thread. Each thread owns 8-element groups tid, tid+256, ...; the loads of four
// groups are issued before any arithmetic so a row's 28 KB is in flight at once.
__device__ inline float router_row_dot(const RouterArgs& a, int e) {
  __shared__ float red[4];
  const int tid = (int)threadIdx.x;
  const size_t D = (size_t)a.D;
  const int esz = a.w_dt == VIB3_DT_F32 ? 4 : 2;
  const char* row = (const char*)a.w + (size_t)e * D * esz;
  float acc = 0.0f;
  const bool vec = (D % 8 == 0) && (((uintptr_t)row & 15) == 0) &&
                   ((((uintptr_t)a.x) & 15) == 0);
  if (vec) {
    const int n8 = (int)(D / 8);
    for (int base = 0; base < n8; base += 4 * 256) {
      float w[4][8], x[4][8];
#pragma unroll
      for (int u = 0; u < 4; u++) {
        const int i = base + u * 256 + tid;
        const int ic = i < n8 ? i : 0;
        load8_stream(row, a.w_dt, (size_t)ic * 8, w[u]);
        load8_act(a.x, a.x_dt, (size_t)ic * 8, x[u]);
      }
#pragma unroll
      for (int u = 0; u < 4; u++) {
        if (base + u * 256 + tid < n8) {
#pragma unroll
          for (int j = 0; j < 8; j++) acc = __builtin_fmaf(x[u][j], w[u][j], acc);
        }
      }
    }
  } else {
    for (size_t d = (size_t)tid; d < D; d += 256)
      acc = __builtin_fmaf(load_act(a.x, a.x_dt, d), load_act(row, a.w_dt, d), acc);
  }
  acc = wave_sum(acc);
  if ((tid & 63) == 0) red[tid >> 6] = acc;
  __syncthreads();
  return (red[0] + red[1]) + (red[2] + red[3]);
}

// The same dot product split in two, so a caller can issue other loads in between: issue()
// starts every load of a row segment (segment `part` of `parts` equal pieces of row e, at most
// 8 * U * 256 elements, 16-byte aligned), finish() waits for them only and reduces the
// segment over the workgroup. The load count does not depend on the dtypes (16-bit rows
// re-read their chunk instead of a second one), so the wait counts stay exact. For parts = 1,
// U = 4 the result is bit for bit that of router_row_dot.
template <int U>
struct RouterSegRaw {
  uint4 w[U][2], x[U][2];
  uint4 n[U];  // RMSNorm weights (f16) of the groups, when the norm is fused
};

// (Evaluated without short-circuits, so every argument it reads is loaded at once.)
__device__ inline bool router_seg_ok(const RouterArgs& a, int parts, int U) {
  return (a.D % (8 * parts) == 0) & (a.D / parts <= 8 * U * 256) &
         ((((uintptr_t)a.w | (uintptr_t)a.x) & 15) == 0) & ((unsigned)a.w_dt <= VIB3_DT_BF16) &
         ((unsigned)a.x_dt <= VIB3_DT_BF16);
}

// NORM: x is the f32 residual stream and the dot product takes RMSNorm(x) (weights nw, the
// inverse RMS given to finish()), element by element as the standalone norm writes it.
template <int U, bool NORM = false>
__device__ inline void router_seg_issue(const RouterArgs& a, int e, int part, int parts,
                                        RouterSegRaw<U>& r, const uint16_t* nw = nullptr) {
  const int tid = (int)threadIdx.x, n8 = a.D / (8 * parts);
  const int wsz = a.w_dt == VIB3_DT_F32 ? 32 : 16, xsz = a.x_dt == VIB3_DT_F32 ? 32 : 16;
  const size_t g0 = (size_t)part * n8;  // first 8-element group of the segment
  const uint8_t* row = (const uint8_t*)a.w + ((size_t)e * (a.D / 8) + g0) * wsz;
  const uint8_t* xs = (const uint8_t*)a.x + g0 * xsz;
#pragma unroll
  for (int u = 0; u < U; u++) {
    const int i = u * 256 + tid;
    const int ic = i < n8 ? i : 0;
    r.w[u][0] = ld_stream(row + (size_t)ic * wsz);
    r.w[u][1] = ld_stream(row + (size_t)ic * wsz + (wsz - 16));
    r.x[u][0] = *(const uint4*)(xs + (size_t)ic * xsz);
    r.x[u][1] = *(const uint4*)(xs + (size_t)ic * xsz + (xsz - 16));
    if (NORM) r.n[u] = *(const uint4*)(nw + (g0 + (size_t)ic) * 8);
  }
}

__device__ inline void raw8(const uint4 (&v)[2], int dt, float* o) {
  if (dt == VIB3_DT_F32) {
    const uint32_t w[8] = {v[0].x, v[0].y, v[0].z, v[0].w, v[1].x, v[1].y, v[1].z, v[1].w};
#pragma unroll
    for (int j = 0; j < 8; j++) o[j] = __uint_as_float(w[j]);
  } else {
    const uint32_t w[4] = {v[0].x, v[0].y, v[0].z, v[0].w};
#pragma unroll
    for (int j = 0; j < 4; j++) {
      const uint16_t lo = (uint16_t)(w[j] & 0xffff), hi = (uint16_t)(w[j] >> 16);
      o[2 * j] = dt == VIB3_DT_F16 ? f16_to_f32(lo) : bf16_to_f32(lo);
      o[2 * j + 1] = dt == VIB3_DT_F16 ? f16_to_f32(hi) : bf16_to_f32(hi);
    }
  }
}

template <int U, bool NORM = false>
__device__ inline float router_seg_finish(const RouterArgs& a, int parts, const RouterSegRaw<U>& r,
                                          float inv = 1.0f) {
  __shared__ float red[4];
  const int tid = (int)threadIdx.x, n8 = a.D / (8 * parts);
  float acc = 0.0f;
#pragma unroll
  for (int u = 0; u < U; u++) {
    if (u * 256 + tid < n8) {
      float w[8], x[8];
      raw8(r.w[u], a.w_dt, w);
      raw8(r.x[u], a.x_dt, x);
      if (NORM) {
        const uint32_t nv[4] = {r.n[u].x, r.n[u].y, r.n[u].z, r.n[u].w};
#pragma unroll
        for (int j = 0; j < 8; j++)
          x[j] = norm_mul(x[j], inv, f16_to_f32((uint16_t)(nv[j >> 1] >> (16 * (j & 1)))));
      }
#pragma unroll
      for (int j = 0; j < 8; j++) acc = __builtin_fmaf(x[j], w[j], acc);
    }
  }
  acc = wave_sum(acc);
  if ((tid & 63) == 0) red[tid >> 6] = acc;
  __syncthreads();
  const float s = (red[0] + red[1]) + (red[2] + red[3]);
  __syncthreads();  // red is reused by the next segment
  return s;
}

}  // namespace vib3
