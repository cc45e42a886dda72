// select.h — top-k expert selection by one wavefront (router scoring of kernels.rs:2307-2440).
//
// Keys are compared as (key desc, index asc): the order a stable descending sort gives, for any
// expert count. The selection runs in one wave; the results land in caller-provided LDS arrays
// (sel[j], wts[j], j < top_k) and, when `publish`, in the router outputs of RouterArgs.
#pragma once

#include "common.h"
#include "kernels.h"
#include "norm.h"

#ifdef VIB3_TRACE_SELECT  // (profiling builds: probes inside the selection too)
#define VIB3_TRACE_FINE(k) VIB3_TRACE_POINT(k)
#else
#define VIB3_TRACE_FINE(k) \
  do {                    \
  } while (0)
#endif

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

// Weights of the selected experts (kernels.rs:2368-2387 softmax, :2389-2436 sigmoid) by the
// whole wave: lane j < top_k handles pick j. Sums run sequentially in pick order (the
// reference's order) through readlane; the per-pick exp and divisions run in parallel.
// sel[j] / selv[j] hold the picks and their values; selv[j] is overwritten by the weight.
__device__ inline void router_weights_wave(const RouterArgs& a, const int* sel, float* selv,
                                           bool publish) {
  const int lane = lane_id();
  const bool mine = lane < a.top_k;
  const float v = mine ? selv[lane] : 0.0f;
  const auto rl = [](float x, int l) {
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), l));
  };
  float w;
  if (a.mode == VIB3_ROUTER_SOFTMAX) {
    float mx = -__builtin_huge_valf();
    for (int j = 0; j < a.top_k; j++) mx = fmaxf(mx, rl(v, j));
    const float e = expf(v - mx);
    float sum = 0.0f;
    for (int j = 0; j < a.top_k; j++) sum += rl(e, j);
    w = e / sum;
  } else {
    w = v;
    if (a.normalize) {
      float total = 0.0f;
      for (int j = 0; j < a.top_k; j++) total += rl(v, j);
      if (total > 1e-20f) w = v / total;
    }
    w *= a.scaling;
  }
  if (mine) {
    selv[lane] = w;
    if (publish) {
      const int id = sel[lane];
      a.ids[lane] = (uint16_t)id;
      a.wts[lane] = w;
      if (a.out_ids) a.out_ids[lane] = (uint16_t)id;
      if (a.out_wts) a.out_wts[lane] = w;
    }
  }
}

// Minimum of an int over the wave (wave-uniform result).
template <int CTRL>
__device__ __forceinline__ int dpp_i(int v) {
  return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xf, 0xf, true);
}
__device__ __forceinline__ int wave_min_i(int v) {
  v = min(v, dpp_i<0xB1>(v));
  v = min(v, dpp_i<0x4E>(v));
  v = min(v, dpp_i<0x141>(v));
  v = min(v, dpp_i<0x140>(v));
  return min(min(__builtin_amdgcn_readlane(v, 0), __builtin_amdgcn_readlane(v, 16)),
             min(__builtin_amdgcn_readlane(v, 32), __builtin_amdgcn_readlane(v, 48)));
}
__device__ __forceinline__ float wave_max_f(float v) {
  v = fmaxf(v, dpp<0xB1>(v));
  v = fmaxf(v, dpp<0x4E>(v));
  v = fmaxf(v, dpp<0x141>(v));
  v = fmaxf(v, dpp<0x140>(v));
  const auto rl = [](float x, int l) {
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), l));
  };
  return fmaxf(fmaxf(rl(v, 0), rl(v, 16)), fmaxf(rl(v, 32), rl(v, 48)));
}

// Top-k by the calling wave (all 64 lanes active). Lane l owns experts l, l+64, ... (R keys);
// each lane first sorts its keys by (key desc, index asc), so the lane heads hold every lane's
// best remaining candidate. A round is then branch-free: the wave maximum of the heads, a
// ballot for the lanes that hold it (the lowest index wins a tie), and the winning lane pops
// its head. The order of the picks is the order of a stable descending sort.
// Fast path for top_k <= 8: no sequential rounds. Let t be the smallest of the eight
// 8-lane-group maxima of the keys; those eight maxima are distinct experts with key >= t, so
// the k-th best key is >= t and every expert of the top-k is a candidate (key >= t). The
// candidates (typically a few dozen) are compacted into LDS, and each candidate's rank is the
// number of candidates that beat it in the (key desc, index asc) order; ranks below k are the
// picks, in order. Returns false (wave-uniformly) when more than 64 candidates pass the bound,
// e.g. with many equal keys; the caller then runs the rounds.
template <int R>
__device__ inline bool select_fast(const RouterArgs& a, const float (&key)[R],
                                   const float (&val)[R], const int (&idx)[R], int* sel,
                                   float* selv) {
  __shared__ __attribute__((aligned(16))) float ck[kWave];
  __shared__ __attribute__((aligned(16))) int ci[kWave];
  __shared__ float cv[kWave];
  constexpr int kNone = 0x7fffffff;
  const int lane = lane_id();
  float m = -__builtin_huge_valf();
#pragma unroll
  for (int r = 0; r < R; r++)
    if (idx[r] != kNone) m = fmaxf(m, key[r]);
  m = fmaxf(m, dpp<0xB1>(m));   // quad_perm [1,0,3,2]
  m = fmaxf(m, dpp<0x4E>(m));   // quad_perm [2,3,0,1]
  m = fmaxf(m, dpp<0x141>(m));  // row_half_mirror: every lane holds its 8-lane group maximum
  float t = __builtin_huge_valf();
#pragma unroll
  for (int g = 0; g < kWave; g += 8)
    t = fminf(t, __int_as_float(__builtin_amdgcn_readlane(__float_as_int(m), g)));
  VIB3_TRACE_FINE(8);  // threshold
  int n = 0;
#pragma unroll
  for (int r = 0; r < R; r++) {
    const bool c = idx[r] != kNone && key[r] >= t;
    const uint64_t mask = __ballot(c);
    const int pos = n + (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(mask >> 32),
                                                       __builtin_amdgcn_mbcnt_lo((uint32_t)mask, 0));
    if (c && pos < kWave) {
      ck[pos] = key[r];
      cv[pos] = val[r];
      ci[pos] = idx[r];
    }
    n += __popcll(mask);
  }
  VIB3_TRACE_VALUE(7, n);
  VIB3_TRACE_FINE(9);  // compacted
  if (n > kWave) return false;
  if (lane >= n && lane < ((n + 7) & ~7)) {  // pad to a multiple of 8: never beats anything
    ck[lane] = -__builtin_huge_valf();
    ci[lane] = kNone;
  }
  wait_lgkm();
  __builtin_amdgcn_wave_barrier();
  // every lane takes candidate `lane` and counts the candidates that beat it, reading the
  // list from LDS eight at a time (broadcast reads, all issued before the compares)
  const float mk = lane < n ? ck[lane] : -__builtin_huge_valf();
  const int mi = lane < n ? ci[lane] : kNone;
  const float mv = lane < n ? cv[lane] : 0.0f;
  int rank = 0;
  for (int j0 = 0; j0 < n; j0 += 8) {
    const float4 ka = *(const float4*)(ck + j0), kb = *(const float4*)(ck + j0 + 4);
    const int4 ia = *(const int4*)(ci + j0), ib = *(const int4*)(ci + j0 + 4);
    const float kk[8] = {ka.x, ka.y, ka.z, ka.w, kb.x, kb.y, kb.z, kb.w};
    const int ii[8] = {ia.x, ia.y, ia.z, ia.w, ib.x, ib.y, ib.z, ib.w};
#pragma unroll
    for (int u = 0; u < 8; u++)  // bitwise, not short-circuit: no branches in the count
      rank += (int)(kk[u] > mk) | ((int)(kk[u] == mk) & (int)(ii[u] < mi));
  }
  if (lane < n && rank < a.top_k) {
    sel[rank] = mi;
    selv[rank] = mv;
  }
  VIB3_TRACE_FINE(10);  // ranked
  wait_lgkm();
  __builtin_amdgcn_wave_barrier();
  return true;
}

// Top-k by the calling wave (all 64 lanes active) from scores already in registers: lane l
// holds the scores of experts l, l+64, ... (sc[r] for expert l + 64r). Each lane first sorts
// its keys by (key desc, index asc), so the lane heads hold every lane's best remaining
// candidate. A round is then branch-free: the wave maximum of the heads, a ballot for the
// lanes that hold it (the lowest index wins a tie), and the winning lane pops its head. The
// order of the picks is the order of a stable descending sort.
// Bias of experts lane, lane + 64, ... (0 without a bias).
template <int R>
__device__ __forceinline__ void load_bias(const RouterArgs& a, float (&bs)[R]) {
#pragma unroll
  for (int r = 0; r < R; r++) bs[r] = a.bias ? a.bias[min(lane_id() + r * kWave, a.E - 1)] : 0.0f;
}

template <int R>
__device__ inline void select_topk_vals(const RouterArgs& a, const float (&sc)[R],
                                        const float (&bs)[R], int* sel, float* selv,
                                        bool publish) {
  const int lane = lane_id();
  constexpr int kNone = 0x7fffffff;
  float key[R], val[R];
  int idx[R];
#pragma unroll
  for (int r = 0; r < R; r++) {
    const int e = lane + r * kWave;
    selection_key(a, sc[r], bs[r], key[r], val[r]);
    if (e >= a.E) key[r] = -__builtin_huge_valf();
    idx[r] = e < a.E ? e : kNone;
  }
  VIB3_TRACE_POINT(5);  // scores and bias in registers
  if (a.top_k <= 8 && select_fast<R>(a, key, val, idx, sel, selv)) {
    VIB3_TRACE_FINE(6);  // picks done
    router_weights_wave(a, sel, selv, publish);
    wait_lgkm();
    __builtin_amdgcn_wave_barrier();
    return;
  }
  // insertion network: R(R-1)/2 compare-exchanges, all lanes in parallel
#pragma unroll
  for (int i = 1; i < R; i++) {
#pragma unroll
    for (int j = i; j > 0; j--) {
      const bool sw = key[j] > key[j - 1] || (key[j] == key[j - 1] && idx[j] < idx[j - 1]);
      const float k0 = key[j - 1], v0 = val[j - 1];
      const int i0 = idx[j - 1];
      key[j - 1] = sw ? key[j] : k0;
      val[j - 1] = sw ? val[j] : v0;
      idx[j - 1] = sw ? idx[j] : i0;
      key[j] = sw ? k0 : key[j];
      val[j] = sw ? v0 : val[j];
      idx[j] = sw ? i0 : idx[j];
    }
  }
  for (int j = 0; j < a.top_k; j++) {
    const float m = wave_max_f(key[0]);
    const bool at_max = key[0] == m;
    const uint64_t holders = __ballot(at_max);
    int win;
    if (__popcll(holders) == 1) {
      win = __builtin_amdgcn_readlane(idx[0], __ffsll((unsigned long long)holders) - 1);
    } else {  // a tie: the lowest index wins (wave-uniform branch)
      win = wave_min_i(at_max ? idx[0] : kNone);
    }
    const bool pop = (win & (kWave - 1)) == lane;
    if (pop) selv[j] = val[0];
    if (lane == 0) sel[j] = win;
#pragma unroll
    for (int r = 0; r + 1 < R; r++) {
      key[r] = pop ? key[r + 1] : key[r];
      val[r] = pop ? val[r + 1] : val[r];
      idx[r] = pop ? idx[r + 1] : idx[r];
    }
    key[R - 1] = pop ? -__builtin_huge_valf() : key[R - 1];
    idx[R - 1] = pop ? kNone : idx[R - 1];
  }
  wait_lgkm();
  __builtin_amdgcn_wave_barrier();
  VIB3_TRACE_FINE(6);  // picks done
  router_weights_wave(a, sel, selv, publish);
  wait_lgkm();
  __builtin_amdgcn_wave_barrier();
}

// Same, loading the scores from memory first.
template <int R>
__device__ inline void select_topk_regs(const RouterArgs& a, const float* scores, int* sel,
                                        float* selv, bool publish) {
  float sc[R], bs[R];
#pragma unroll
  for (int r = 0; r < R; r++) sc[r] = scores[min(lane_id() + r * kWave, a.E - 1)];
  load_bias<R>(a, bs);
  select_topk_vals<R>(a, sc, bs, sel, selv, publish);
}

// Wait until every expert's logit of this launch is published in `slots` (one 64-bit word per
// expert: generation tag << 32 | f32 bits, written with a device-scope atomic store by the
// workgroup that computed it), then select. Tags make the wait independent of any ordering
// between different addresses, so no device-wide fence is needed. The wait is bounded: after
// RouterArgs::spin_limit polls (kRouterSpinLimit normally) the wave records an error, which
// the host reads with vib3_moe_int4_layer_status, computes the logits it has not seen from the
// router weights, and selects from the complete set.

#ifndef VIB3_POLL_GAP
#define VIB3_POLL_GAP 20  // s_sleep units (64 clocks) between the two poll rounds in flight
#endif
constexpr int kPollGap = VIB3_POLL_GAP;

// Logit of router row e computed by one wave (64 lanes over d, then a wave sum), for a wait
// that gave up: x is the router's activation, or RMSNorm(x) with weights nw and inverse RMS
// inv (the fused sublayer prologue). Its summation order is not the workgroup's, so the value
// can differ from the published one in the last bits.
__device__ inline float wave_row_dot(const RouterArgs& a, int e, const uint16_t* nw, float inv) {
  const int lane = lane_id();
  const size_t row = (size_t)e * a.D;
  float acc = 0.0f;
  for (int d = lane; d < a.D; d += kWave) {
    float x = load_act(a.x, a.x_dt, d);
    if (nw) x = norm_mul(x, inv, f16_to_f32(nw[d]));
    acc = __builtin_fmaf(x, load_act(a.w, a.w_dt, row + d), acc);
  }
  return wave_sum(acc);
}

template <int R>
__device__ inline void select_topk_published(const RouterArgs& a, int* sel, float* selv,
                                             bool publish, const uint16_t* nw = nullptr,
                                             float inv = 1.0f) {
  const int lane = lane_id();
  float sc[R], bs[R];
  load_bias<R>(a, bs);  // before the wait, off the critical path
  // Two poll rounds in flight, the second issued about half a round trip after the first,
  // so the last logit is seen about a quarter of a round trip sooner on average.
  uint64_t va[R], vb[R];
  const uint32_t want = a.gen ^ a.poll_xor;
  auto issue = [&](uint64_t (&v)[R]) {
#pragma unroll
    for (int r = 0; r < R; r++)
      v[r] = __hip_atomic_load(a.slots + min(lane + r * kWave, a.E - 1), __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
  };
  auto ready = [&](const uint64_t (&v)[R]) {
    bool ok = true;
#pragma unroll
    for (int r = 0; r < R; r++) ok &= (uint32_t)(v[r] >> 32) == want;
    return __all(ok);
  };
  auto take = [&](const uint64_t (&v)[R]) {
#pragma unroll
    for (int r = 0; r < R; r++) sc[r] = __uint_as_float((uint32_t)v[r]);
  };
  uint32_t missing = 0;  // bit r: this lane's expert lane + 64 r was never published
  issue(va);
  __builtin_amdgcn_s_sleep(kPollGap);
  issue(vb);
  for (int it = 0;; it += 2) {
    if (ready(va)) {
      take(va);
      break;
    }
    if (it >= a.spin_limit) {
      // The wait gave up (reported through the status word): the logits not yet published
      // are computed here from the router weights, so the selection still sees every expert
      // and every workgroup selects the same ones.
      if (lane == 0) a.error[0] = 1;
      take(va);
#pragma unroll
      for (int r = 0; r < R; r++)
        missing |= (lane + r * kWave < a.E && (uint32_t)(va[r] >> 32) != want) ? 1u << r : 0u;
      break;
    }
    issue(va);
    if (ready(vb)) {
      take(vb);
      break;
    }
    issue(vb);
  }
  if (__ballot(missing != 0)) {
#pragma unroll
    for (int r = 0; r < R; r++) {
      uint64_t m = __ballot((missing >> r) & 1u);
      while (m) {
        const int l = (int)__builtin_ctzll(m);
        m &= m - 1;
        const float v = wave_row_dot(a, l + r * kWave, nw, inv);
        if (lane == l) sc[r] = v;
      }
    }
  }
  select_topk_vals<R>(a, sc, bs, sel, selv, publish);
}

__device__ inline void select_topk_published_small(const RouterArgs& a, int* sel, float* selv,
                                                   bool publish, const uint16_t* nw = nullptr,
                                                   float inv = 1.0f) {
  if (a.E <= 2 * kWave) select_topk_published<2>(a, sel, selv, publish, nw, inv);
  else if (a.E <= 4 * kWave) select_topk_published<4>(a, sel, selv, publish, nw, inv);
  else if (a.E <= 6 * kWave) select_topk_published<6>(a, sel, selv, publish, nw, inv);
  else select_topk_published<8>(a, sel, selv, publish, nw, inv);
}

// Register selection for up to 8 * 64 experts, with the register count matched to E.
__device__ inline void select_topk_small(const RouterArgs& a, const float* scores, int* sel,
                                         float* selv, bool publish) {
  if (a.E <= 2 * kWave) select_topk_regs<2>(a, scores, sel, selv, publish);
  else if (a.E <= 4 * kWave) select_topk_regs<4>(a, scores, sel, selv, publish);
  else if (a.E <= 6 * kWave) select_topk_regs<6>(a, scores, sel, selv, publish);
  else select_topk_regs<8>(a, scores, sel, selv, publish);
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
  wait_lgkm();
  __builtin_amdgcn_wave_barrier();
  router_weights_wave(a, sel, selv, publish);
  wait_lgkm();
  __builtin_amdgcn_wave_barrier();
}

}  // namespace vib3
