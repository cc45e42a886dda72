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
#include "router_dot.h"
#include "select.h"

namespace vib3 {

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
