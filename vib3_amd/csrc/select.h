// select.h — top-k expert selection by one wavefront (router scoring of kernels.rs:2307-2440).
//
// Keys are compared as (key desc, index asc): the order a stable descending sort gives, for any
// expert count. The selection runs in one wave; the results land in caller-provided LDS arrays
// (sel[j], wts[j], j < top_k) and, when `publish`, in the router outputs of RouterArgs.
#pragma once

#include "common.h"
#include "kernels.h"

namespace vib3 {

// (key, index) arg-max over the wave: larger key wins, ties go to the lower index (the order
// of a stable descending sort). DPP inside each 16-lane row, then the four row winners.
__device__ __forceinline__ void better(float& k, int& i, float ok, int oi) {
  if (ok > k || (ok == k && oi < i)) { k = ok; i = oi; }
}

template <int CTRL>
__device__ __forceinline__ void argmax_step(float& k, int& i) {
  const float ok = __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(k), CTRL, 0xf, 0xf, false));
  const int oi = __builtin_amdgcn_mov_dpp(i, CTRL, 0xf, 0xf, false);
  better(k, i, ok, oi);
}

__device__ __forceinline__ int wave_argmax(float k, int i) {
  argmax_step<0xB1>(k, i);   // quad_perm [1,0,3,2]
  argmax_step<0x4E>(k, i);   // quad_perm [2,3,0,1]
  argmax_step<0x141>(k, i);  // row_half_mirror
  argmax_step<0x140>(k, i);  // row_mirror
  float bk = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(k), 0));
  int bi = __builtin_amdgcn_readlane(i, 0);
#pragma unroll
  for (int r = 16; r < 64; r += 16) {
    better(bk, bi, __int_as_float(__builtin_amdgcn_readlane(__float_as_int(k), r)),
           __builtin_amdgcn_readlane(i, r));
  }
  return bi;
}

__device__ __forceinline__ void selection_key(const RouterArgs& a, float s, float bias, float& key,
                                              float& val) {
  val = s;
  key = s;
  if (a.mode == VIB3_ROUTER_SIGMOID) {
    val = 1.0f / (1.0f + expf(-s));
    key = val + bias;
  }
  if (key != key) key = -__builtin_huge_valf();  // NaN ranks last
}

// Weights of the selected experts (kernels.rs:2368-2387 softmax, :2389-2436 sigmoid), computed
// sequentially by lane 0 from the selected values; selv[j] is overwritten by the weight.
__device__ inline void router_weights_lane0(const RouterArgs& a, const int* sel, float* selv,
                                            bool publish) {
  float mx = -__builtin_huge_valf(), sum = 0.0f, total = 0.0f;
  if (a.mode == VIB3_ROUTER_SOFTMAX) {
    for (int j = 0; j < a.top_k; j++) mx = fmaxf(mx, selv[j]);
    for (int j = 0; j < a.top_k; j++) sum += expf(selv[j] - mx);
  } else if (a.normalize) {
    for (int j = 0; j < a.top_k; j++) total += selv[j];
  }
  for (int j = 0; j < a.top_k; j++) {  // in place: each weight depends only on its own value
    float w;
    if (a.mode == VIB3_ROUTER_SOFTMAX) {
      w = expf(selv[j] - mx) / sum;
    } else {
      w = selv[j];
      if (a.normalize && total > 1e-20f) w /= total;
      w *= a.scaling;
    }
    selv[j] = w;
    if (publish) {
      a.ids[j] = (uint16_t)sel[j];
      a.wts[j] = w;
      if (a.out_ids) a.out_ids[j] = (uint16_t)sel[j];
      if (a.out_wts) a.out_wts[j] = w;
    }
  }
}

// Top-k by the calling wave (all 64 lanes). Keys live in registers: lane l owns experts
// l, l+64, ...; each round is a local arg-max over R registers and one wave arg-max.
template <int R>
__device__ inline void select_topk_regs(const RouterArgs& a, const float* scores, int* sel,
                                        float* selv, bool publish) {
  const int lane = lane_id();
  float key[R], val[R], sc[R], bs[R];
  const float* bp = a.bias ? a.bias : scores;
#pragma unroll
  for (int r = 0; r < R; r++) {  // all loads first: one round trip, not R
    const int e = min(lane + r * kWave, a.E - 1);
    sc[r] = scores[e];
    bs[r] = bp[e];
  }
#pragma unroll
  for (int r = 0; r < R; r++) {
    const int e = lane + r * kWave;
    selection_key(a, sc[r], a.bias ? bs[r] : 0.0f, key[r], val[r]);
    if (e >= a.E) key[r] = -__builtin_huge_valf();
  }
  unsigned taken = 0;  // bit r: expert lane + 64r already selected
  for (int j = 0; j < a.top_k; j++) {
    float bk = -__builtin_huge_valf();
    int bi = 0x7fffffff;
#pragma unroll
    for (int r = 0; r < R; r++) {
      const int e = lane + r * kWave;
      if (e < a.E && !(taken >> r & 1u)) better(bk, bi, key[r], e);
    }
    const int win = wave_argmax(bk, bi);
    if ((win & (kWave - 1)) == lane) {
#pragma unroll
      for (int r = 0; r < R; r++)
        if (r == (win >> 6)) selv[j] = val[r];
      taken |= 1u << (win >> 6);
    }
    if (lane == 0) sel[j] = win;
  }
  __builtin_amdgcn_s_waitcnt(0);
  __builtin_amdgcn_wave_barrier();
  if (lane == 0) router_weights_lane0(a, sel, selv, publish);
  __builtin_amdgcn_s_waitcnt(0);
  __builtin_amdgcn_wave_barrier();
}

// Same selection for up to kMaxExperts experts with the keys in LDS.
__device__ inline void select_topk_lds(const RouterArgs& a, const float* scores, int* sel,
                                       float* selv, bool publish) {
  __shared__ float key[kMaxExperts];
  __shared__ float val[kMaxExperts];
  const int lane = lane_id();
  __shared__ unsigned char taken[kMaxExperts];
  for (int e = lane; e < a.E; e += kWave) {
    selection_key(a, scores[e], a.bias ? a.bias[e] : 0.0f, key[e], val[e]);
    taken[e] = 0;
  }
  for (int j = 0; j < a.top_k; j++) {
    float bk = -__builtin_huge_valf();
    int bi = 0x7fffffff;
    for (int e = lane; e < a.E; e += kWave)
      if (!taken[e]) better(bk, bi, key[e], e);
    const int win = wave_argmax(bk, bi);
    if ((win & (kWave - 1)) == lane) {  // only the owning lane touches an expert's entries
      selv[j] = val[win];
      taken[win] = 1;
    }
    if (lane == 0) sel[j] = win;
  }
  __builtin_amdgcn_s_waitcnt(0);
  __builtin_amdgcn_wave_barrier();
  if (lane == 0) router_weights_lane0(a, sel, selv, publish);
  __builtin_amdgcn_s_waitcnt(0);
  __builtin_amdgcn_wave_barrier();
}

}  // namespace vib3
