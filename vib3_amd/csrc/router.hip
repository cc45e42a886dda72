// router.hip — MoE router for batch-1 decode on gfx950.
//
// Logits: one 256-thread workgroup per expert row; each thread reads 8 consecutive weights per
// step with 16-byte loads (f32 rows: two loads), the wave reduces with DPP, four wave sums are
// combined in a fixed order. Selection: one wavefront holds the scores in LDS and picks the
// top-k by k rounds of a wave-wide (key desc, index asc) arg-max (select.h) — stable-sort order
// of the reference (kernels.rs:2370, :2416) for any expert count up to 4096, unlike the
// power-of-two bitonic sort of kernels.cu:4011. Inside the fused MoE layer the selection runs
// in the prologue of the gate/up kernel instead of a launch of its own.
#include <math.h>

#include "common.h"
#include "kernels.h"
#include "select.h"

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
__device__ float router_row_dot(const RouterArgs& a, int e) {
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

__global__ __launch_bounds__(256) void k_router_logits(RouterArgs a) {
  const float s = router_row_dot(a, (int)blockIdx.x);
  if (threadIdx.x == 0) a.scores[blockIdx.x] = s;
}

template <bool REGS>
__global__ __launch_bounds__(64) void k_router_select(RouterArgs a) {
  __shared__ int sel[64];
  __shared__ float wts[64];
  if (REGS) select_topk_small(a, a.scores, sel, wts, true);
  else select_topk_lds(a, a.scores, sel, wts, true);
}

int launch_router_logits(const RouterArgs& a, hipStream_t s, KTime t) {
  hipExtLaunchKernelGGL(k_router_logits, dim3((unsigned)a.E), dim3(256), 0, s, t.start, t.stop, 0, a);
  VIB3_RETURN_LAUNCH();
}

int launch_router_select(const RouterArgs& a, hipStream_t s, KTime t) {
  if (a.E <= 8 * kWave)
    hipExtLaunchKernelGGL(k_router_select<true>, dim3(1), dim3(64), 0, s, t.start, t.stop, 0, a);
  else
    hipExtLaunchKernelGGL(k_router_select<false>, dim3(1), dim3(64), 0, s, t.start, t.stop, 0, a);
  VIB3_RETURN_LAUNCH();
}

}  // namespace vib3
