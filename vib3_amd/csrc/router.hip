// router.hip — MoE router for batch-1 decode on gfx950.
//
// Logits: one 256-thread workgroup per expert row; each thread reads 8 consecutive weights per
// step with 16-byte loads (f32 rows: two loads), the wave reduces with DPP, four wave sums are
// combined in a fixed order. Selection: one wavefront holds the scores in LDS and picks the
// top-k by k rounds of a wave-wide (key desc, index asc) arg-max — stable-sort order of the
// reference (kernels.rs:2370, :2416) for any expert count up to 4096, unlike the power-of-two
// bitonic sort of kernels.cu:4011. The fused launch lets the last workgroup to finish its
// logit (completion counter, release/acquire fences) run the selection, so routing costs one
// launch and no host synchronisation.
#include <math.h>

#include "common.h"
#include "kernels.h"

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
// valid in thread 0.
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
    const size_t n8 = D / 8;
#pragma unroll 4
    for (size_t i = (size_t)tid; i < n8; i += 256) {
      float w[8], x[8];
      load8_stream(row, a.w_dt, i * 8, w);
      load8_act(a.x, a.x_dt, i * 8, x);
#pragma unroll
      for (int j = 0; j < 8; j++) acc = __builtin_fmaf(x[j], w[j], acc);
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

// Top-k selection by wave 0 of the calling workgroup (64 threads participate).
__device__ void router_select_wave(const RouterArgs& a, const float* scores) {
  __shared__ float key[kMaxExperts];
  __shared__ float val[kMaxExperts];
  __shared__ unsigned char taken[kMaxExperts];
  __shared__ int sel[64];
  const int lane = lane_id();
  const int E = a.E;
  for (int e = lane; e < E; e += kWave) {
    const float s = scores[e];
    float v = s, k = s;
    if (a.mode == VIB3_ROUTER_SIGMOID) {
      v = 1.0f / (1.0f + expf(-s));
      k = a.bias ? v + a.bias[e] : v;
    }
    if (k != k) k = -__builtin_huge_valf();  // NaN ranks last
    key[e] = k;
    val[e] = v;
    taken[e] = 0;
  }
  __builtin_amdgcn_s_waitcnt(0);
  __builtin_amdgcn_wave_barrier();
  for (int j = 0; j < a.top_k; j++) {
    float bk = -__builtin_huge_valf();
    int bi = 0x7fffffff;
    for (int e = lane; e < E; e += kWave) {
      if (taken[e]) continue;
      const float k = key[e];
      if (k > bk || (k == bk && e < bi)) { bk = k; bi = e; }
    }
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
      const float ok = __shfl_xor(bk, off);
      const int oi = __shfl_xor(bi, off);
      if (ok > bk || (ok == bk && oi < bi)) { bk = ok; bi = oi; }
    }
    if (lane == (bi & 63)) taken[bi] = 1;
    if (lane == 0) sel[j] = bi;
    __builtin_amdgcn_s_waitcnt(0);
    __builtin_amdgcn_wave_barrier();
  }
  if (lane != 0) return;
  // Weights (kernels.rs:2368-2387 softmax, :2389-2436 sigmoid), sequential like the reference.
  float w[64];
  if (a.mode == VIB3_ROUTER_SOFTMAX) {
    float mx = -__builtin_huge_valf();
    for (int j = 0; j < a.top_k; j++) mx = fmaxf(mx, val[sel[j]]);
    float sum = 0.0f;
    for (int j = 0; j < a.top_k; j++) sum += expf(val[sel[j]] - mx);
    for (int j = 0; j < a.top_k; j++) w[j] = expf(val[sel[j]] - mx) / sum;
  } else {
    for (int j = 0; j < a.top_k; j++) w[j] = val[sel[j]];
    if (a.normalize) {
      float total = 0.0f;
      for (int j = 0; j < a.top_k; j++) total += w[j];
      if (total > 1e-20f)
        for (int j = 0; j < a.top_k; j++) w[j] /= total;
    }
    for (int j = 0; j < a.top_k; j++) w[j] *= a.scaling;
  }
  for (int j = 0; j < a.top_k; j++) {
    a.ids[j] = (uint16_t)sel[j];
    a.wts[j] = w[j];
    if (a.out_ids) a.out_ids[j] = (uint16_t)sel[j];
    if (a.out_wts) a.out_wts[j] = w[j];
  }
}

__global__ __launch_bounds__(256) void k_router_logits(RouterArgs a) {
  const float s = router_row_dot(a, (int)blockIdx.x);
  if (threadIdx.x == 0) a.scores[blockIdx.x] = s;
}

__global__ __launch_bounds__(64) void k_router_select(RouterArgs a) { router_select_wave(a, a.scores); }

__global__ __launch_bounds__(256) void k_router_fused(RouterArgs a) {
  __shared__ int is_last;
  const float s = router_row_dot(a, (int)blockIdx.x);
  if (threadIdx.x == 0) {
    a.scores[blockIdx.x] = s;
    __threadfence();  // release the logit before counting this workgroup as done
    const unsigned prev = atomicAdd(a.counter, 1u);
    is_last = prev == gridDim.x - 1;
  }
  __syncthreads();
  if (!is_last) return;
  __threadfence();  // acquire every other workgroup's logit
  if (threadIdx.x < 64) {
    router_select_wave(a, a.scores);
    if (threadIdx.x == 0) atomicExch(a.counter, 0u);  // ready for the next launch
  }
}

int launch_router_fused(const RouterArgs& a, hipStream_t s) {
  hipLaunchKernelGGL(k_router_fused, dim3((unsigned)a.E), dim3(256), 0, s, a);
  VIB3_RETURN_LAUNCH();
}

int launch_router_logits(const RouterArgs& a, hipStream_t s) {
  hipLaunchKernelGGL(k_router_logits, dim3((unsigned)a.E), dim3(256), 0, s, a);
  VIB3_RETURN_LAUNCH();
}

int launch_router_select(const RouterArgs& a, hipStream_t s) {
  hipLaunchKernelGGL(k_router_select, dim3(1), dim3(64), 0, s, a);
  VIB3_RETURN_LAUNCH();
}

}  // namespace vib3
