// norm.h — pieces of the pre-MoE RMSNorm (vib3_rms_norm_f32, kernels.cu:921-955) shared by
// the standalone prologue kernel and the gate/up kernel that fuses it.
//
// Thread t of a 256-thread workgroup accumulates x[d]^2 for d = t, t + 256, ... with fused
// multiply-adds, the 256 partials are summed by a halving tree, then rms = sqrt(ss / D + eps)
// and inv = 1 / rms (both correctly rounded); y[d] = (x[d] * inv) * w[d] with two rounded
// products. Every workgroup that follows this order computes the same inverse RMS, bit for bit.
#pragma once

#include "common.h"

namespace vib3 {

constexpr int kNormMax = 32;  // elements per thread: D <= 256 * kNormMax

// Inverse RMS from each thread's partial sum (the halving tree over the workgroup's 256
// threads; every thread gets the result).
__device__ inline float block_inv_rms(float p, int D, float eps) {
  __shared__ float ss[256];
  const int tid = (int)threadIdx.x;
  ss[tid] = p;
  __syncthreads();
  if (tid < 128) ss[tid] += ss[tid + 128];
  __syncthreads();
  if (tid < 64) {
    // the steps s = 64 .. 1 in the first wave's registers: lane t adds lane t + s, the same
    // pairs as the tree in memory (lanes >= s compute values no later step reads)
    float v = ss[tid] + ss[tid + 64];
#pragma unroll
    for (int s = 32; s > 0; s >>= 1) v += __shfl_down(v, s);
    if (tid == 0) ss[0] = v;
  }
  __syncthreads();
  const float rms = sqrtf(ss[0] / (float)D + eps);
  const float inv = 1.0f / rms;
  __syncthreads();  // ss is reused by the next call
  return inv;
}

__device__ __forceinline__ float norm_mul(float x, float inv, float w) {
#pragma clang fp contract(off)
  return x * inv * w;
}

}  // namespace vib3
