// kernels.h — argument blocks and internal launchers shared by the .hip translation units.
#pragma once

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "common.h"
#include "../../include/vib3_hip.h"

namespace vib3 {

// Optional timing of one launch: events recorded by the dispatch itself at kernel begin / end
// (hipExtLaunchKernel), so the interval is the kernel's own duration on its stream.
struct KTime {
  hipEvent_t start = nullptr, stop = nullptr;
};

// Router: logits (one workgroup per expert) and top-k selection (one wavefront, select.h).
struct RouterArgs {
  const void* x;
  int x_dt;
  const void* w;
  int w_dt;
  const float* bias;
  int D, E, top_k, mode;
  float scaling;
  int normalize;
  float* scores;       // [E] logits
  uint16_t* ids;       // [top_k] selection (workspace)
  float* wts;          // [top_k]
  uint16_t* out_ids;   // optional copies for the caller
  float* out_wts;
  // logits published in the gate/up kernel (fused routing): tagged slots, see select.h
  uint64_t* slots;     // [E]
  // Tag of this launch's slots (never 0). With gen_word set, the tag lives on the device:
  // the gate/up kernel uses next_tag(*gen_word) and the layer's down kernel stores that value
  // back, so every launch (also every replay of a captured graph) publishes under a new tag.
  // Without gen_word, `gen` is the tag (stage-by-stage timing launches).
  uint32_t gen;
  uint32_t* gen_word;
  uint32_t poll_xor;   // 0; nonzero only in the forced-timeout test (no slot ever matches)
  int spin_limit;      // polls before the wait gives up
  int* error;          // set to 1 if a wait gave up
};

// Polls of the fused router's bounded wait before it gives up, records an error and computes
// the logits it has not seen itself (a poll round is one device round trip, ~1-2 us, so the
// limit is tens of milliseconds; a wait normally ends within a few rounds).
constexpr int kRouterSpinLimit = 1 << 15;

// Device tags are 31-bit and never 0; host-side stage tags set bit 31, so the two never meet.
__host__ __device__ inline uint32_t next_tag(uint32_t g) {
  const uint32_t n = (g + 1) & 0x7fffffffu;
  return n ? n : 1u;
}

int launch_router_logits(const RouterArgs& a, hipStream_t s, KTime t = {});
int launch_router_select(const RouterArgs& a, hipStream_t s, KTime t = {});

enum { kRouteGiven = 0, kRouteScores = 1, kRouteFused = 2 };

// Experts whose selection fits the register path of select.h (8 keys per lane).
constexpr int kMaxExpertsInKernel = 8 * 64;
// Rows of one matrix (or of the up/gate pair) per expert slot. Slot s of a paged launch reads
// expert ids[s] from routed_table for s < top_k and shared expert s - top_k from shared_table;
// a flat launch (routed_table == nullptr, one slot) reads flat0 / flat1.
struct RowsArgs {
  const void* x;
  int x_dt;
  int K, M, g, sdt;
  int nslots;
  const uint64_t* routed_table;
  const uint64_t* shared_table;
  const uint16_t* ids;
  int top_k;
  int max_pages;
  int rpp[3];
  uint64_t magic[3];  // page_magic(rpp[s])
  MatRef flat0, flat1;
  void* out;
  int out_dt;
  size_t out_stride;  // elements between slots in out
  int KS;             // waves that split one row's k range (set by the launcher)
  int RPT;            // rows per team
  // route = kRouteGiven: slots take experts from `ids`. kRouteScores: every workgroup selects
  // the top-k of router.scores in its prologue (wave 0; block 0 also publishes router.ids /
  // router.wts). kRouteFused: workgroups first compute the router logits themselves (block b
  // takes experts b, b + grid, ...), publish them as tagged slots, and then select as above.
  int route;
  RouterArgs router;
  // f32 activations of a paged launch as int16 block fixed point (one integer dot product per
  // weight pair, error 2^-16 of each 32-chunk's largest value) instead of the hi + lo split
  int x_i16;
  // paged launches that route: block 0 also writes the down segment's page addresses of every
  // slot here ([nslots][down_pages], slot order), for the down kernel that follows (or null)
  uint64_t* down_bases;
  int down_pages;
  // fused routing with shared experts: stream the shared items on the workgroups without a
  // router row while the routing is pending (the launcher clears it where it does not apply)
  int pre_shared;
  // fused sublayer prologue (fused routing, f32 x): x and router.x are the residual stream,
  // which the kernel normalises (RMSNorm, weights norm_w); the second wave of workgroup s
  // also stores shared expert s's sigmoid gate (gate_w row s . RMSNorm(x)) in shared_w[s]
  const uint16_t* norm_w;
  float eps;
  const uint16_t* gate_w;
  int ngate;
  float* shared_w;
};

// Down projection of every slot for a block of RB output rows plus the weighted expert sum.
struct DownArgs {
  const void* h;  // [nslots][K] intermediate, f16 or f32
  int h_dt;
  int K, M, g, sdt;
  int nslots;
  const uint64_t* routed_table;
  const uint64_t* shared_table;
  const uint16_t* ids;
  // page addresses of the down segment per slot ([nslots][bases_stride], written by the
  // gate/up kernel of the same layer call), or null: the kernel reads the page tables itself
  const uint64_t* bases;
  int bases_stride;
  const float* wts;
  int top_k;
  int max_pages;
  int rpp;  // rows per page of the down segment
  uint64_t magic;  // page_magic(rpp)
  int KS;
  int RB;
  int round_f16;
  float* out;
  const float* residual;  // out = residual + sum, or null
  const float* shared_w;  // [nslots - top_k] weights of the shared experts, or null (1.0)
  uint32_t* gen_word;     // router tag word advanced by block 0 (fused routing), or null
};

// The down kernel, the layer's last, advances the router tag for the next launch. It runs
// after the gate/up kernel on the same stream, so no launch still reads the old value.
__device__ inline void advance_router_tag(uint32_t* gen_word) {
  if (gen_word && blockIdx.x == 0 && threadIdx.x == 0) *gen_word = next_tag(*gen_word);
}

struct GenericArgs {
  const void* x;
  int x_dt;
  int K, M, g, sdt;
  const uint8_t* data0;
  const uint16_t* scales0;
  const uint8_t* data1;
  const uint16_t* scales1;
  void* out;
  int out_dt;
};

int launch_rows(RowsArgs a, bool dual, hipStream_t s, KTime t = {});
// whether launch_rows(a) lists the down page addresses at a.down_bases (when given)
bool rows_write_bases(const RowsArgs& a);
// whether launch_rows(a) fuses the RMSNorm / shared-gate prologue given in a.norm_w ...
bool rows_fuse_prologue(const RowsArgs& a);
int launch_down(DownArgs a, hipStream_t s, KTime t = {});
int launch_generic(GenericArgs a, bool dual, hipStream_t s);
// RMSNorm of x into xn (norm_w set) and the shared experts' sigmoid gates (gate_w set).
int launch_moe_prologue(const void* x, int x_dt, const uint16_t* norm_w, float eps, int D,
                        float* xn, const uint16_t* gate_w, int ns, float* shared_w,
                        hipStream_t st);

constexpr int kMaxExperts = 4096;

// Resident workgroups per CU for a kernel at a block size, and the CU count (cached per device;
// plain host queries, no allocation).
static inline int device_cus() {
  static int cus[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (!cus[dev]) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
      n = 256;
    cus[dev] = n;
  }
  return cus[dev];
}

template <typename K>
static inline int resident_blocks(K kernel, int block) {
  int per_cu = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kernel, block, 0) != hipSuccess ||
      per_cu <= 0)
    per_cu = 1;
  return per_cu * device_cus();
}


}  // namespace vib3
