// int4_gemv.hip — batch-1 INT4 GEMV kernels for gfx950 (MI355X).
//
// Decode is HBM-bound: every weight byte is read once per token. The kernels therefore
//  * stream weights with 16-byte non-temporal loads (one 32-column chunk per lane),
//  * keep the activation slice of each lane in VGPRs for the whole launch (a lane always owns
//    the same chunk columns, so the activations are loaded and converted once),
//  * dequantise in registers with v_dot2_f32_f16 on masked nibbles (see chunk_dot),
//  * reduce each row across the wave with DPP + readlane, never through LDS,
//  * resolve page-table indirection with one table read per row (scalar load).
//
// k_int4_rows      — rows of one or two matrices per expert slot (fused gate/up + SwiGLU, or a
//                    single GEMV), used by the layer and by the partial_* launchers.
// k_down_combine   — down projection of all expert slots for a block of output rows, with the
//                    weighted sum over experts (fixed order, no atomics) in the epilogue.
// k_int4_generic   — any k (including odd k) and unaligned pointers; one wave per row.
#include <stdlib.h>

#include "common.h"
#include "kernels.h"
#include "norm.h"
#include "router_dot.h"
#include "select.h"

namespace vib3 {

// ------------------------------------------------------------------------- row dot products
//
// A row batch = U rows of one matrix (or of the up/gate pair). issue() starts every 16-byte
// load of the batch; reduce() does the arithmetic and the wave sums. Keeping the two apart lets
// the loops start the next batch's loads before reducing the current one.

template <int NCH, bool DUAL, int U>
struct RowBatch {
  uint4 w0[U][NCH], w1[U][NCH];
  uint16_t q0[U][NCH], q1[U][NCH];
};

// Data and scale rows of row r of a paged matrix whose page (r's) starts at `base`.
__device__ __forceinline__ void page_row(const uint8_t* base, int r, int rpp, int rows,
                                         uint64_t magic, int pk, int ng, const uint8_t*& d,
                                         const uint16_t*& s) {
  const int p = (int)(((uint64_t)(uint32_t)r * magic) >> 32);
  const int rr = r - p * rpp;
  const int rows_here = min(rpp, rows - p * rpp);
  d = base + (size_t)rr * pk;
  s = (const uint16_t*)(base + (size_t)rows_here * pk) + (size_t)rr * ng;
}

template <bool PAGED, int NCH, bool DUAL, int U>
__device__ __forceinline__ void issue(RowBatch<NCH, DUAL, U>& b, const MatRef& m0, const MatRef& m1,
                                      const int (&ra)[U], const int (&cidx)[NCH],
                                      const int (&gidx)[NCH], int pk, int ng, int cpr,
                                      const void* dummy = nullptr) {
#pragma unroll
  for (int u = 0; u < U; u++) {
    const uint8_t *d0, *d1 = nullptr;
    const uint16_t *s0, *s1 = nullptr;
    mat_row<PAGED>(m0, ra[u], pk, ng, d0, s0);
    if (DUAL) mat_row<PAGED>(m1, ra[u], pk, ng, d1, s1);
    if (dummy) {  // a batch past the end: the same loads from a small cached buffer, no branch
      d0 = d1 = (const uint8_t*)dummy;
      s0 = s1 = (const uint16_t*)dummy;
    }
#pragma unroll
    for (int j = 0; j < NCH; j++) {
      // lanes past the last chunk re-read it (no divergent branch around the loads); their
      // activation chunk is zero, so they add nothing
      const int c = min(cidx[j], cpr - 1);
      const uint32_t off = (uint32_t)c * 16u;  // 32-bit lane offset on a uniform row base
      b.w0[u][j] = ld_stream(d0 + off);
      b.q0[u][j] = ld_u16(s0 + gidx[j]);
      if (DUAL) {
        b.w1[u][j] = ld_stream(d1 + off);
        b.q1[u][j] = ld_u16(s1 + gidx[j]);
      }
    }
  }
}

// Wave-uniform sums (scaled back by 2^24) of the batch's rows.
template <int NCH, bool DUAL, int XM, int U>
__device__ __forceinline__ void reduce(const RowBatch<NCH, DUAL, U>& b, const XChunk (&xh)[NCH],
                                       const XChunk (&xl)[NCH], const int (&cidx)[NCH], int cpr,
                                       int sdt, float (&t0)[U], float (&t1)[U]) {
#pragma unroll
  for (int u = 0; u < U; u++) {
    float acc0 = 0.f, acc1 = 0.f;
#pragma unroll
    for (int j = 0; j < NCH; j++) {
      float p0 = XM == kXi16 ? chunk_dot_i16(b.w0[u][j], xh[j], xl[j].xs8)
                             : chunk_dot(b.w0[u][j], xh[j]);
      if (XM == kXsplit) p0 += chunk_dot(b.w0[u][j], xl[j]);
      acc0 = __builtin_fmaf(p0, decode_scale(b.q0[u][j], sdt), acc0);
      if (DUAL) {
        float p1 = XM == kXi16 ? chunk_dot_i16(b.w1[u][j], xh[j], xl[j].xs8)
                               : chunk_dot(b.w1[u][j], xh[j]);
        if (XM == kXsplit) p1 += chunk_dot(b.w1[u][j], xl[j]);
        acc1 = __builtin_fmaf(p1, decode_scale(b.q1[u][j], sdt), acc1);
      }
    }
    t0[u] = wave_sum(acc0) * kTwo24;
    t1[u] = DUAL ? wave_sum(acc1) * kTwo24 : 0.f;
  }
}

template <bool PAGED, int NCH, bool DUAL, int XM, int U>
__device__ __forceinline__ void dot_rows(const MatRef& m0, const MatRef& m1, const int (&ra)[U],
                                         const XChunk (&xh)[NCH], const XChunk (&xl)[NCH],
                                         const int (&cidx)[NCH], const int (&gidx)[NCH], int pk,
                                         int ng, int cpr, int sdt, float (&t0)[U], float (&t1)[U]) {
  RowBatch<NCH, DUAL, U> b;
  issue<PAGED, NCH, DUAL, U>(b, m0, m1, ra, cidx, gidx, pk, ng, cpr);
  reduce<NCH, DUAL, XM, U>(b, xh, xl, cidx, cpr, sdt, t0, t1);
}

// Chunk indices of this lane: chunk c = (ks * NCH + j) * 64 + lane and its scale group.
template <int NCH>
__device__ __forceinline__ void chunk_index(int ks, int g, int cpr, int (&cidx)[NCH],
                                            int (&gidx)[NCH]) {
  const int lane = lane_id();
#pragma unroll
  for (int j = 0; j < NCH; j++) {
    cidx[j] = (ks * NCH + j) * kWave + lane;
    gidx[j] = (min(cidx[j], cpr - 1) * 32) / g;
  }
}

// Activation chunks of this lane (see chunk_index), converted to f16 pairs.
template <int NCH, int XM>
__device__ __forceinline__ void load_x(const void* x, int x_dt, int cpr, const int (&cidx)[NCH],
                                       XChunk (&xh)[NCH], XChunk (&xl)[NCH],
                                       const uint16_t* nw = nullptr, float inv = 1.0f) {
#pragma unroll
  for (int j = 0; j < NCH; j++) {
    if (cidx[j] < cpr) {
      float xv[32];
      load_chunk_act(x, x_dt, cidx[j], xv);
      if (XM == kXi16n) {  // RMSNorm(x), element by element as the standalone norm writes it
        const uint4* np = (const uint4*)(nw + 32 * (size_t)cidx[j]);
#pragma unroll
        for (int i = 0; i < 4; i++) {
          const uint4 v = np[i];
          const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
          for (int k = 0; k < 8; k++)
            xv[8 * i + k] = norm_mul(xv[8 * i + k], inv,
                                     f16_to_f32((uint16_t)(w[k >> 1] >> (16 * (k & 1)))));
        }
      }
      if (XM == kXi16 || XM == kXi16n) {
        make_chunk_i16(xv, xh[j], xl[j]);
      } else {
        make_chunk(xv, xh[j], xl[j]);
        if (XM != kXsplit) zero_chunk(xl[j]);
      }
    } else {
      zero_chunk(xh[j]);
      zero_chunk(xl[j]);
    }
  }
}

// Page-table rows of one slot's segment: routed slot s < top_k is expert `expert`, the others
// are shared experts s - top_k; flat launches use flat0 / flat1.
__device__ __forceinline__ MatRef slot_matrix(const RowsArgs& a, int slot, int expert, int seg,
                                              int which) {
  if (!a.routed_table) return which == 0 ? a.flat0 : a.flat1;  // flat launch
  const uint64_t* t;
  if (slot < a.top_k) t = a.routed_table + ((size_t)expert * 3 + seg) * a.max_pages;
  else t = a.shared_table + ((size_t)(slot - a.top_k) * 3 + seg) * a.max_pages;
  return MatRef{t, nullptr, nullptr, a.rpp[seg], a.M, a.magic[seg]};
}

__device__ __forceinline__ float rows_epilogue(bool dual, float up, float gate) {
  // DUAL: matrix 0 = up (segment 0), matrix 1 = gate (segment 1); SiLU goes on the gate.
  return dual ? (gate / (1.0f + expf(-gate))) * up : up;
}

__device__ __forceinline__ void store_out(const RowsArgs& a, size_t o, float v) {
  if (a.out_dt == VIB3_DT_F16) ((uint16_t*)a.out)[o] = f32_to_f16_bits(v);
  else ((float*)a.out)[o] = v;
}

// ------------------------------------------------------------------------- k_int4_rows
//
// KS == 1 (k <= 8192): every wave owns whole rows. Work items are (slot, row pair) and waves
// stride over them (grid sized to the resident capacity), so all CUs stay busy to the end.
// KS > 1: the KS waves of a team split one row's k range and combine through LDS.


#ifndef VIB3_X_SHARED
#define VIB3_X_SHARED 2  // (build-time switch: one wave converts the activations for all four;
                         // 2 = only for f32 activations)
#endif

template <int NCH, bool DUAL, int XM, bool PAGED>
__global__ __launch_bounds__(256) void k_int4_rows(RowsArgs a) {
  VIB3_TRACE_POINT(0);
  // Fused routing: this workgroup's router row (blockIdx.x < E) is on every routed row's
  // critical path, so its loads are the kernel's first, ahead of the item bookkeeping and its
  // kernel-argument reads. Fused prologue (NORM): the residual stream in the norm's thread
  // layout (x[t + 256 i]) goes out just before it; the launcher guarantees fused routing with
  // every router row in the split form below, and K <= 256 * kNormMax.
  if (PAGED)  // (the arguments that choose and address it, requested in one round trip)
    asm volatile("" ::"s"(a.route), "s"(a.router.E), "s"(a.router.D), "s"(a.router.w),
                 "s"(a.router.x), "s"(a.router.w_dt), "s"(a.router.x_dt));
  const bool fused = PAGED && a.route == kRouteFused;
  const int E = a.router.E, G = (int)gridDim.x;
  constexpr bool NORM = XM == kXi16n;
  float xr[NORM ? kNormMax : 1];
  if (NORM) {
#pragma unroll
    for (int i = 0; i < kNormMax; i++) {
      const int d = (int)threadIdx.x + 256 * i;
      xr[i] = ((const float*)a.x)[d < a.K ? d : 0];
    }
  }
  const bool split_row = fused & ((int)blockIdx.x < E) & router_seg_ok(a.router, 1, 4);
  RouterSegRaw<4> rrow;
  if (split_row) router_seg_issue<4, NORM>(a.router, (int)blockIdx.x, 0, 1, rrow, a.norm_w);
  VIB3_TRACE_POINT(11);  // router row issued
  const int lane = lane_id();
  const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));  // wave-uniform (SGPR)
  const int pk = a.K / 2, ng = (a.K + a.g - 1) / a.g, cpr = a.K / 32;
  XChunk xh[NCH], xl[NCH];
  int cidx[NCH], gidx[NCH];

  // Items are (slot, row), shared-expert slots first; waves stride over them.
  __shared__ int s_sel[64];
  __shared__ float s_wts[64];
  // per slot: page-table row of each matrix (resolved once; a 16-bit id load in the loop
  // would be a vector load whose wait drains all prefetched weight loads)
  __shared__ const uint64_t* s_tab[16][2];
  __shared__ int s_xready;  // the second wave's activation copy is in LDS (pre-streaming)
  chunk_index<NCH>(0, a.g, cpr, cidx, gidx);
  const int items = a.nslots * a.M;
  const int stride = (int)gridDim.x * 4;
  const int M = a.M, nslots = a.nslots, top_k = a.top_k;
  const int rpp0 = a.rpp[0], rpp1 = a.rpp[1];
  const uint64_t magic0 = a.magic[0], magic1 = a.magic[1];
  // item = q * M + row; q maps to a slot with the shared experts first
  const int it0 = (int)blockIdx.x * 4 + wave;
  auto slot_of = [&](int q) {  // q < nslots; shared slots (>= top_k) come first
    if (nslots == top_k) return q;
    const int v = q + top_k;
    return v >= nslots ? v - nslots : v;
  };
  // A wave's items. Normally item k is it0 + k * stride. With a.pre_shared (fused routing with
  // shared experts; set by the launcher), the shared-expert items [0, S) go to waves 1-3 of
  // every workgroup, which stream them while wave 0 waits for the routing (after their
  // workgroup's router row), and every wave takes the routed items S + it0 + k * stride after
  // them: the stream that waits for the selection is one item shorter.
  // Workgroups b and b + G/2 share a CU (dispatch order). Where both compute a router row
  // (E > G/2), the second one selects on its third wave (the first selects on wave 0: the two
  // selections run on different SIMDs) and takes no shared items before the selection (its
  // polls then do not queue behind six streaming waves); the shared items go to the others.
  const int Gh = G / 2;
  const bool two_router = fused && E > Gh;
  const bool second = (int)blockIdx.x >= Gh;
  const int selw = (two_router && second) ? 2 : 0;   // the selecting wave
  const int pw = wave < selw ? wave : wave - 1;       // rank among the other three
  const bool no_pre = two_router && second && (int)blockIdx.x < E;
  const int nwg = two_router ? Gh + max(0, G - E) : G;  // workgroups taking shared items
  const int rk = (two_router && second) ? (int)blockIdx.x - (E - Gh) : (int)blockIdx.x;
  const int NP = nwg * 3, S = (nslots - top_k) * M;
  const bool pre = a.pre_shared && wave != selw && !no_pre;
  const int u = rk * 3 + pw;
  const int cs = pre ? max(0, (S - u + NP - 1) / max(NP, 1)) : 0;  // this wave's shared items
  const int rbase = a.pre_shared ? S + it0 : it0;
  auto item_at = [&](int k) { return k < cs ? u + k * NP : rbase + (k - cs) * stride; };
  auto shared_table_of = [&](int slot, int which) {
    return a.shared_table + ((size_t)(slot - top_k) * 3 + which) * a.max_pages;
  };
  // Lane k of this wave holds its k-th item's row and page-table rows (filled after routing);
  // the loop fetches them with v_readlane: no memory access, so no wait can drain the
  // prefetched weight loads.
  int my_row = 0;
  uint64_t my_t0 = 0, my_t1 = 0;
  RowBatch<NCH, DUAL, 1> buf[2];
  // start() is issued unconditionally, also for a batch past the last item (its loads then
  // read the activation vector). A branch around the loads would leave the compiler unsure
  // how many loads are in flight.
  auto start = [&](RowBatch<NCH, DUAL, 1>& buf, int k, bool direct, int item,
                   bool dummy = false) {
    const bool past = dummy || item >= items;
    MatRef m0, m1;
    int row;
    if (PAGED) {
      const uint64_t* t0;
      const uint64_t* t1;
      if (direct) {  // first item, shared expert: straight from the kernel arguments
        const int q = item / M;
        row = item - q * M;
        t0 = shared_table_of(slot_of(q), 0);
        t1 = shared_table_of(slot_of(q), 1);
      } else {
        if (past) k -= 1;  // any valid lane; the loads go to the activation vector instead
        k &= kWave - 1;
        row = __builtin_amdgcn_readlane(my_row, k);
        t0 = (const uint64_t*)(uintptr_t)(
            ((uint64_t)(uint32_t)__builtin_amdgcn_readlane((int)(my_t0 >> 32), k) << 32) |
            (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)my_t0, k));
        t1 = (const uint64_t*)(uintptr_t)(
            ((uint64_t)(uint32_t)__builtin_amdgcn_readlane((int)(my_t1 >> 32), k) << 32) |
            (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)my_t1, k));
      }
      m0 = MatRef{t0, nullptr, nullptr, rpp0, M, magic0};
      m1 = DUAL ? MatRef{t1, nullptr, nullptr, rpp1, M, magic1} : m0;
    } else {
      row = min(item, items - 1);  // flat launches have one slot
      m0 = a.flat0;
      m1 = a.flat1;
    }
    const int ra[1] = {row};
    // a batch past the end reads the (cached) activation vector: no HBM traffic
    issue<PAGED, NCH, DUAL, 1>(buf, m0, m1, ra, cidx, gidx, pk, ng, cpr, past ? a.x : nullptr);
    // keep the scheduler from sinking these loads below the previous batch's arithmetic
    __builtin_amdgcn_sched_barrier(0);
  };
  // Results stay in lanes (lane k holds this wave's k-th item; the launcher keeps k < 64)
  // and are stored after the loop: a store inside it would share the load counter and make
  // the waits drain the prefetched loads.
  float res = 0.f;
  int kres = 0;
  auto finish = [&](const RowBatch<NCH, DUAL, 1>& buf) {
    float t0[1], t1[1];
    reduce<NCH, DUAL, (XM == kXi16n ? kXi16 : XM), 1>(buf, xh, xl, cidx, cpr, a.sdt, t0, t1);
    const float v = rows_epilogue(DUAL, t0[0], t1[0]);
    if (lane == kres) res = v;
    kres++;
  };
  const bool have = item_at(0) < items;
  if (PAGED && wave == selw && lane < nslots && lane >= top_k) {
    s_tab[lane][0] = shared_table_of(lane, 0);
    s_tab[lane][1] = shared_table_of(lane, 1);
  }
  // a shared-expert row needs no routing: start its loads before the selection
  const bool early = have && PAGED && !a.pre_shared && slot_of(it0 / M) >= top_k;
  // Fused routing: workgroup b computes router rows b, b + grid, ... and publishes each as a
  // tagged slot. The first row's loads go out before anything else, and a workgroup computing
  // a router row starts its expert stream only after the selection, so the CU's memory
  // pipeline serves the router rows, which every routed row waits for, first. (Cutting rows
  // into halves to spread them evenly over the two workgroups of a CU measured slower.)
  auto publish = [&](int e, float v) {
    if (threadIdx.x == 0) {
      __hip_atomic_store(a.router.slots + e,
                         ((uint64_t)a.router.gen << 32) | __float_as_uint(v), __ATOMIC_RELAXED,
                         __HIP_MEMORY_SCOPE_AGENT);
      if (a.router.scores) a.router.scores[e] = v;
    }
  };
  // one wave converts the activations for the workgroup (through LDS) for f32 activations;
  // with f16 / bf16 (an exact permutation) every wave converts its own (measured faster)
  constexpr bool XSH = VIB3_X_SHARED == 1 || (VIB3_X_SHARED == 2 && XM != kXf16);
  if (XSH && a.pre_shared) {  // (LDS holds whatever the CU's last workgroup left)
    if (threadIdx.x == 0) s_xready = 0;
    __syncthreads();
  }
  // this launch's tag, read once the router row's loads are out
  if (fused && a.router.gen_word) a.router.gen = next_tag(*a.router.gen_word);
  const bool early_now = early && !(fused && (int)blockIdx.x < E);
  if (early_now) start(buf[0], 0, true, it0);
  float inv = 1.0f;
  if (NORM) {
    float p = 0.0f;
#pragma unroll
    for (int i = 0; i < kNormMax; i++) {
      const float v = (int)threadIdx.x + 256 * i < a.K ? xr[i] : 0.0f;
      p = __builtin_fmaf(v, v, p);
    }
    inv = block_inv_rms(p, a.K, a.eps);
  }
  if (fused) {
    int e = (int)blockIdx.x;
    if (split_row) {
      publish(e, router_seg_finish<4, NORM>(a.router, 1, rrow, inv));
      VIB3_TRACE_POINT(12);  // router row published
      e += G;
    }
    for (; e < E; e += G) {  // more rows than workgroups: one at a time
      publish(e, router_row_dot(a.router, e));
      __syncthreads();  // router_row_dot's reduction buffer is reused by the next row
    }
  }
  if (NORM && wave == 2 && (int)blockIdx.x < a.ngate) {
    // Shared expert s = block's gate, by the block's third wave while the first selects and
    // the second loads the activations:
    // sigmoid(gate_w[s] . RMSNorm(x)) as the prologue kernel computes it (thread t of 256
    // accumulates elements t + 256 i in i order, each wave's partials summed by wave_sum, the
    // four wave sums pairwise); this one wave plays the four waves' threads in turn.
    const uint16_t* gw = a.gate_w + (size_t)blockIdx.x * a.K;
    float ws0 = 0.0f, ws1 = 0.0f, ws2 = 0.0f, ws3 = 0.0f;
#pragma unroll 1
    for (int vw = 0; vw < 4; vw++) {
      const int t = vw * kWave + lane;
      float acc = 0.0f;
#pragma unroll
      for (int h = 0; h < kNormMax; h += kNormMax / 2) {  // (half the loads at a time)
        uint16_t gr[kNormMax / 2], nr[kNormMax / 2];
        float xg[kNormMax / 2];
#pragma unroll
        for (int i = 0; i < kNormMax / 2; i++) {
          const int d = min(t + 256 * (h + i), a.K - 1);
          gr[i] = gw[d];
          nr[i] = a.norm_w[d];
          xg[i] = ((const float*)a.x)[d];
        }
#pragma unroll
        for (int i = 0; i < kNormMax / 2; i++) {
          const bool in = t + 256 * (h + i) < a.K;
          const float xn = norm_mul(in ? xg[i] : 0.0f, inv, f16_to_f32(nr[i]));
          acc = __builtin_fmaf(xn, in ? f16_to_f32(gr[i]) : 0.0f, acc);
        }
      }
      const float v = wave_sum(acc);
      ws0 = vw == 0 ? v : ws0;
      ws1 = vw == 1 ? v : ws1;
      ws2 = vw == 2 ? v : ws2;
      ws3 = vw == 3 ? v : ws3;
    }
    if (lane == 0) {
      const float g = (ws0 + ws1) + (ws2 + ws3);
      a.shared_w[blockIdx.x] = 1.0f / (1.0f + expf(-g));
    }
  }
  // The activation chunks, while the routing is pending. A lane's chunks depend on the lane
  // only, so every wave of the workgroup holds the same ones: the second wave loads and
  // converts them and the others copy them from LDS after the barrier below (a quarter of
  // the cache traffic, and none of it ahead of the selecting wave's polls).
  constexpr int XQ = XM == kXi16n ? kXi16 : XM;
  constexpr int XLW = XQ == kXsplit ? 17 : XQ == kXi16 ? 1 : 0;  // words of xl kept
  __shared__ uint32_t s_x[NCH * (17 + XLW) * kWave];
  auto copy_x = [&]() {  // this wave's chunks from the second wave's LDS copy
#pragma unroll
    for (int j = 0; j < NCH; j++) {
      XWords hw, lw{};
#pragma unroll
      for (int k = 0; k < 17; k++) hw.w[k] = s_x[(j * (17 + XLW) + k) * kWave + lane];
#pragma unroll
      for (int k = 0; k < XLW; k++)
        lw.w[XLW == 1 ? 16 : k] = s_x[(j * (17 + XLW) + 17 + k) * kWave + lane];
      xh[j] = __builtin_bit_cast(XChunk, hw);
      xl[j] = __builtin_bit_cast(XChunk, lw);
    }
  };
  if (!XSH || wave == 1) {
    load_x<NCH, XM>(a.x, a.x_dt, cpr, cidx, xh, xl, a.norm_w, inv);
#pragma unroll
    for (int j = 0; j < NCH; j++) {
      const auto hw = __builtin_bit_cast(XWords, xh[j]);
      const auto lw = __builtin_bit_cast(XWords, xl[j]);
#pragma unroll
      for (int k = 0; k < 17; k++) s_x[(j * (17 + XLW) + k) * kWave + lane] = hw.w[k];
#pragma unroll
      for (int k = 0; k < XLW; k++)
        s_x[(j * (17 + XLW) + 17 + k) * kWave + lane] = lw.w[XLW == 1 ? 16 : k];
    }
    // waves that stream shared items before the barrier take the copy once this flag is set
    if (XSH && a.pre_shared) {
      wait_lgkm();
      if (lane == 0) __hip_atomic_store(&s_xready, 1, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
    }
  }
  VIB3_TRACE_POINT(1);
  if (PAGED && top_k > 0 && wave == selw) {
    // the selection is on every routed row's critical path: issue ahead of the streaming
    // waves that share this SIMD
    __builtin_amdgcn_s_setprio(3);
    if (a.route == kRouteFused) {
      select_topk_published_small(a.router, s_sel, s_wts, blockIdx.x == 0,
                                  NORM ? a.norm_w : nullptr, inv);
    } else if (a.route == kRouteScores) {
      select_topk_small(a.router, a.router.scores, s_sel, s_wts, blockIdx.x == 0);
    } else if (lane < top_k) {
      s_sel[lane] = a.ids[lane];
    }
    wait_lgkm();
    __builtin_amdgcn_wave_barrier();
    if (lane < top_k) {
      const uint64_t* rt = a.routed_table + (size_t)s_sel[lane] * 3 * a.max_pages;
      s_tab[lane][0] = rt;
      s_tab[lane][1] = rt + a.max_pages;
    }
    __builtin_amdgcn_s_setprio(0);
    VIB3_TRACE_POINT(2);
  }
  if (pre && cs > 0) {
    if (XSH && wave != 1) {  // (the second wave sets the flag without waiting)
      while (__hip_atomic_load(&s_xready, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_WORKGROUP) == 0)
        __builtin_amdgcn_s_sleep(1);
      copy_x();
    }
    // the shared items, straight from the kernel arguments, while the routing is pending;
    // the same two-buffer pipeline as the loop below, the step after the last one a dummy
    start(buf[0], 0, true, item_at(0));
    for (int k = 0;; k += 2) {
      bool done = false;
#pragma unroll
      for (int b = 0; b < 2; b++) {
        const int ahead = k + b + 1;
        __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
        start(buf[(b + 1) % 2], ahead, true, item_at(min(ahead, cs - 1)), ahead >= cs);
        finish(buf[b]);
        if (ahead >= cs) {
          done = true;
          break;
        }
      }
      if (done) break;
    }
    VIB3_TRACE_POINT(13);  // shared items done
  }
  __syncthreads();
  VIB3_TRACE_POINT(3);
  if (XSH && wave != 1 && !(pre && cs > 0)) copy_x();
  // The down segment's page addresses of every slot, for the down kernel (one table round
  // trip there less): wave 0 of workgroup b reads entries 64 b + lane (+ 64 G ...) of the
  // [slot][page] list. The first entry's load goes out beside the wave's first item and is
  // stored after the loop, so it costs no wait of its own.
  typedef __attribute__((address_space(1))) const uint64_t gtab;
  const int npl = PAGED && a.down_bases ? a.nslots * a.down_pages : 0;
  auto pl_entry = [&](int i) {
    const int sl = i / a.down_pages, p = i - sl * a.down_pages;
    const uint64_t* t = sl < top_k ? a.routed_table + ((size_t)s_sel[sl] * 3 + 2) * a.max_pages
                                   : a.shared_table + ((size_t)(sl - top_k) * 3 + 2) * a.max_pages;
    return t + p;
  };
  const int pl_i = wave == selw ? (int)blockIdx.x * kWave + lane : npl;
  uint64_t pl_v = 0;
  if (pl_i < npl) {
    for (int i = pl_i + G * kWave; i < npl; i += G * kWave) a.down_bases[i] = *(gtab*)pl_entry(i);
    pl_v = *(gtab*)pl_entry(pl_i);
  }
  auto pl_store = [&]() {
    if (pl_i < npl) a.down_bases[pl_i] = pl_v;
  };
  if (!have) {
    pl_store();
    return;
  }
  if (item_at(cs) >= items) {  // shared items only: store them
    if (lane < kres) {
      const int item = item_at(lane), q = item / M;
      store_out(a, (size_t)slot_of(q) * a.out_stride + (item - q * M), res);
    }
    pl_store();
    return;
  }
  if (PAGED) {
    // lane k <- this wave's k-th item (lanes past the end keep a valid page-table row)
    const int item = min(item_at(lane), items - 1);
    {
      const int q = item / M;
      my_row = item - q * M;
      const int slot = slot_of(q);
      my_t0 = (uint64_t)(uintptr_t)s_tab[slot][0];
      my_t1 = (uint64_t)(uintptr_t)s_tab[slot][1];
    }
  }
  if (!early_now) start(buf[0], cs, false, item_at(cs));
  // Two buffers: item k + 1's loads go out, then item k is reduced. Each step first takes
  // delivery of everything in flight, so a wave has one item's loads (8 KB for a gate/up row
  // pair of k = 7168) outstanding at a time: streaming measured fastest with about that much
  // in flight per wave (two items per wave in flight, or a third buffer, measured slower).
  // The explicit wait also makes the step independent of how the compiler counts loads at
  // the loop head.
  for (int k = cs;; k += 2) {
    bool done = false;
#pragma unroll
    for (int b = 0; b < 2; b++) {
      const int ahead = k + b + 1;
      __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
      start(buf[(b + 1) % 2], ahead, false, item_at(ahead));
      finish(buf[b]);
      if (item_at(ahead) >= items) {
        done = true;
        break;
      }
    }
    if (done) break;
  }
  if (lane < kres) {
    const int item = item_at(lane);
    const int q = item / M;
    store_out(a, (size_t)slot_of(q) * a.out_stride + (item - q * M), res);
  }
  pl_store();
  VIB3_TRACE_POINT(4);
}

template <int NCH, bool DUAL, int XM, bool PAGED>
__global__ __launch_bounds__(256) void k_int4_rows_ksplit(RowsArgs a) {
  const int lane = lane_id();
  const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));  // wave-uniform (SGPR)
  const int pk = a.K / 2, ng = (a.K + a.g - 1) / a.g, cpr = a.K / 32;
  XChunk xh[NCH], xl[NCH];
  int cidx[NCH], gidx[NCH];

  const int ks = wave % a.KS;
  const int team = wave / a.KS;
  const int teams = 4 / a.KS;
  const int slot = (int)blockIdx.y;
  const int r0 = ((int)blockIdx.x * teams + team) * a.RPT;
  const int nrows = max(0, min(a.RPT, a.M - r0));
  const int e = (PAGED && slot < a.top_k) ? (int)a.ids[slot] : 0;
  const MatRef m0 = slot_matrix(a, slot, e, 0, 0);
  const MatRef m1 = DUAL ? slot_matrix(a, slot, e, 1, 1) : m0;
  chunk_index<NCH>(ks, a.g, cpr, cidx, gidx);
  load_x<NCH, XM>(a.x, a.x_dt, cpr, cidx, xh, xl);
  float res0 = 0.f, res1 = 0.f;
  for (int i = 0; i < nrows; i += 2) {
    const int ra[2] = {r0 + i, i + 1 < nrows ? r0 + i + 1 : r0 + i};
    float t0[2], t1[2];
    dot_rows<PAGED, NCH, DUAL, XM, 2>(m0, m1, ra, xh, xl, cidx, gidx, pk, ng, cpr, a.sdt, t0, t1);
    if (lane == i) { res0 = t0[0]; res1 = t1[0]; }
    if (lane == i + 1) { res0 = t0[1]; res1 = t1[1]; }
  }
  __shared__ float part0[4][kWave];
  __shared__ float part1[4][kWave];
  part0[wave][lane] = res0;
  part1[wave][lane] = res1;
  __syncthreads();
  if (ks != 0) return;
  res0 = 0.f;
  res1 = 0.f;
  for (int q = 0; q < a.KS; q++) {
    res0 += part0[team * a.KS + q][lane];
    res1 += part1[team * a.KS + q][lane];
  }
  if (lane < nrows)
    store_out(a, (size_t)slot * a.out_stride + r0 + lane, rows_epilogue(DUAL, res0, res1));
}

// ------------------------------------------------------------------------- k_down_combine
//
// Down projection of every expert slot for blocks of RB output rows, plus the weighted expert
// sum. A row is handled by 16 lanes (4 rows per wave instruction): lane `sub` of a 16-lane group
// owns chunks sub + 16 j (j < 4) of the wave's k range, so one 16-byte load per lane per j
// reads four 256-byte row segments, and a row's sum needs only 4 DPP steps inside the group
// (no cross-row readlanes). One workgroup = nslots * KS waves (slot, k part); per-row sums meet
// in LDS and wave 0 forms sum_s w_s * f16(d_s) in slot order (router order, then shared).

constexpr int kDownJ = 4;        // chunks per lane per row
constexpr int kDownRows = 4;     // rows per wave instruction (64 lanes / 16)
constexpr int kDownSpan = 16 * kDownJ;  // chunks of one k part

// Sum over each 16-lane row of the wave; every lane gets its row's total.
__device__ __forceinline__ float row16_sum(float v) {
  v += dpp<0xB1>(v);
  v += dpp<0x4E>(v);
  v += dpp<0x141>(v);
  v += dpp<0x140>(v);
  return v;
}

template <int U>
struct DownBatch {
  uint4 w[U][kDownJ];
  uint16_t q[U][kDownJ];
};

// WIDE: up to 16 waves per workgroup (VGPRs capped at 128: one 4-row group per batch);
// otherwise up to 10 waves with two 4-row groups (8 KB per wave) per batch.
template <bool SPLIT, bool WIDE>
__global__ __launch_bounds__(WIDE ? 1024 : 640) void k_down_combine(DownArgs a) {
  constexpr int U = 1;  // one 4-row group per batch (two batches in flight)
  const int lane = lane_id();
  const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
  const int slot = wave / a.KS;
  const int ks = wave - slot * a.KS;
  const int grp = lane >> 4, sub = lane & 15;
  const int pk = a.K / 2, ng = (a.K + a.g - 1) / a.g, cpr = a.K / 32;

  // the slot's expert id is a 16-bit (vector) load: make the table row wave-uniform once
  const int expert = slot < a.top_k ? __builtin_amdgcn_readfirstlane((int)a.ids[slot]) : 0;
  const uint64_t* t = slot < a.top_k
                          ? a.routed_table + ((size_t)expert * 3 + 2) * a.max_pages
                          : a.shared_table + ((size_t)(slot - a.top_k) * 3 + 2) * a.max_pages;
  const MatRef m{uniform_ptr(t), nullptr, nullptr, a.rpp, a.M, a.magic};

  // this lane's chunks (clamped for the loads; chunks past the end get a zero activation)
  int cidx[kDownJ], cld[kDownJ], gidx[kDownJ];
#pragma unroll
  for (int j = 0; j < kDownJ; j++) {
    cidx[j] = ks * kDownSpan + sub + 16 * j;
    cld[j] = min(cidx[j], cpr - 1);
    gidx[j] = (cld[j] * 32) / a.g;
  }
  const char* hbase = (const char*)a.h + (size_t)slot * a.K * (a.h_dt == VIB3_DT_F32 ? 4 : 2);

  __shared__ float part[16][kWave];
  const int blocks = (a.M + a.RB - 1) / a.RB;
  if ((int)blockIdx.x >= blocks) return;
  constexpr int RPB = kDownRows * U;            // rows per batch
  const int ipb = (a.RB + RPB - 1) / RPB;       // batches per block
  const int my_blocks = (blocks - (int)blockIdx.x + (int)gridDim.x - 1) / (int)gridDim.x;
  const int n = my_blocks * ipb;
  struct Pos { int bb, i0; };
  auto advance = [&](Pos p) {
    p.i0 += RPB;
    if (p.i0 >= ipb * RPB) { p.i0 = 0; p.bb += (int)gridDim.x; }
    return p;
  };
  // start() runs unconditionally (see k_int4_rows); a batch past the end is given the position
  // fetched just before it (rows clamp to M - 1, so every position is a valid one)
  auto start = [&](DownBatch<U>& b, Pos p) {
    const int r0 = p.bb * a.RB, nr = min(a.RB, a.M - r0);
#pragma unroll
    for (int u = 0; u < U; u++) {
      // the four rows of a batch are wave-uniform values: resolve each with a scalar table
      // read, then every 16-lane group picks its own
      const uint8_t* d = nullptr;
      const uint16_t* sc = nullptr;
#pragma unroll
      for (int q = 0; q < kDownRows; q++) {
        const int r = r0 + min(p.i0 + u * kDownRows + q, nr - 1);
        const uint8_t* dq;
        const uint16_t* sq;
        mat_row<true>(m, r, pk, ng, dq, sq);
        if (grp == q) { d = dq; sc = sq; }
      }
#pragma unroll
      for (int j = 0; j < kDownJ; j++) {
        b.w[u][j] = ld_stream(d + (size_t)cld[j] * 16);
        b.q[u][j] = ld_u16(sc + gidx[j]);
      }
    }
    // keep the scheduler from sinking these loads below the previous batch's arithmetic
    __builtin_amdgcn_sched_barrier(0);
  };
  // router weights: lane s holds slot s's (read once; a load at each block's combine would
  // wait for every weight load in flight)
  const float my_w = lane < a.top_k    ? a.wts[lane]
                     : lane < a.nslots ? (a.shared_w ? a.shared_w[lane - a.top_k] : 1.0f)
                                       : 0.f;
  XChunk xh[kDownJ], xl[kDownJ];
  auto finish = [&](const DownBatch<U>& b, Pos p) {
    const int r0 = p.bb * a.RB, nr = min(a.RB, a.M - r0);
#pragma unroll
    for (int u = 0; u < U; u++) {
      float acc = 0.f;
#pragma unroll
      for (int j = 0; j < kDownJ; j++) {
        float pj = chunk_dot(b.w[u][j], xh[j]);
        if (SPLIT) pj += chunk_dot(b.w[u][j], xl[j]);
        acc = __builtin_fmaf(pj, decode_scale(b.q[u][j], a.sdt), acc);
      }
      const float sum = row16_sum(acc) * kTwo24;
      const int i = p.i0 + u * kDownRows + grp;
      if (sub == 0 && i < kWave) part[wave][i] = sum;
    }
    if (p.i0 + RPB >= ipb * RPB) {
      // block complete: combine the slots' rows
      __syncthreads();
      if (wave == 0 && lane < nr) {
        // weighted_accumulate_f32 over the slots in router order, then the shared experts
        // with weight 1.0 or their sigmoid gate (engine.rs:5262-5302, :6392-6451):
        // o = o + w * d with separate roundings.
        float o = 0.0f;
        for (int s = 0; s < a.nslots; s++) {
          float d = 0.0f;
          for (int q = 0; q < a.KS; q++) d += part[s * a.KS + q][lane];
          if (a.round_f16) d = (float)(half_t)d;
          const float w = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(my_w), s));
          o = add_mul_rn(o, w, d);
        }
        // the residual add after the sublayer (engine.rs:5302)
        a.out[r0 + lane] = a.residual ? a.residual[r0 + lane] + o : o;
      }
      __syncthreads();
    }
  };
  DownBatch<U> A, B;
  Pos q0{(int)blockIdx.x, 0};
  Pos q1 = advance(q0);
  start(A, q0);
  // activations: the 4 chunks of h this lane multiplies, loaded after the first weights
#pragma unroll
  for (int j = 0; j < kDownJ; j++) {
    if (cidx[j] < cpr) {
      float xv[32];
      load_chunk_act(hbase, a.h_dt, cidx[j], xv);
      make_chunk(xv, xh[j], xl[j]);
      if (!SPLIT) zero_chunk(xl[j]);
    } else {
      zero_chunk(xh[j]);
      zero_chunk(xl[j]);
    }
  }
  for (int k = 0;; k += 2) {
    start(B, k + 1 >= n ? q0 : q1);
    finish(A, q0);
    if (k + 1 >= n) break;
    q0 = advance(q1);
    start(A, k + 2 >= n ? q1 : q0);
    finish(B, q1);
    if (k + 2 >= n) break;
    q1 = advance(q0);
  }
  advance_router_tag(a.gen_word);
}

// ------------------------------------------------------------------------- k_down_rows
//
// Down projection + weighted combine with the activations of every slot staged once per
// workgroup in LDS, already in chunk_dot's pair layout (so a batch costs no conversion work).
// A wave owns a group of R output rows (64 / R lanes per row, J chunks per lane per pass) and
// walks the slots in router order, each slot in ceil(chunks / (64 / R * J)) passes over k, so
// the combine o = o + w_s * d_s happens in registers in the reference's order: no cross-wave
// reduction, no barrier in the loop. f16 intermediates whose staged form fits 64 KB of LDS;
// other shapes use k_down_combine.

template <int J>
struct DownRowsBatch {
  uint4 w[J];
  uint16_t q[J];
};

// Sum over each run of L lanes (L = 16, 32 or 64); every lane gets its run's total.
template <int L>
__device__ __forceinline__ float lanes_sum(float v) {
  v = row16_sum(v);
  if (L >= 32) v += __shfl_xor(v, 16);
  if (L >= 64) v += __shfl_xor(v, 32);
  return v;
}

#ifndef VIB3_DOWN_SCALAR_PAGES
#define VIB3_DOWN_SCALAR_PAGES 1  // (build-time switch of the scalar page-address path)
#endif
constexpr int kDownScalarSlots = 16;  // most slots whose page addresses k_down_rows keeps in SGPRs

template <int R, int J, int NB, bool ONE>  // ONE: the whole row in one pass (cpr <= CPP)
__global__ __launch_bounds__(512) void k_down_rows(DownArgs a) {
  VIB3_TRACE_POINT(0);
  extern __shared__ uint4 lds[];
  constexpr int L = kWave / R;  // lanes per row
  constexpr int CPP = L * J;    // chunks per pass
  const int lane = lane_id();
  const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
  const int grp = lane / L, sub = lane % L;
  const int cpr = a.K / 32, pk = a.K / 2, ng = (a.K + a.g - 1) / a.g;
  const int P = ONE ? 1 : (cpr + CPP - 1) / CPP;  // passes per slot
  const int ns = a.nslots, top_k = a.top_k;
  const int CT = ONE ? CPP : cpr;  // chunks per slot in LDS (one pass: zero past cpr)
  uint4* xq = lds;                                       // [ns][4][CT] pair words
  float* xsum = (float*)(lds + (size_t)ns * 4 * CT);     // [ns][CT] offset term

  const int G = (a.M + R - 1) / R;  // row groups
  const int g0 = (int)blockIdx.x * (int)(blockDim.x >> 6) + wave;
  // scale index of chunk c: (32 c) / g, a shift for the usual power-of-two group sizes
  const bool g_pow2 = (a.g & (a.g - 1)) == 0;
  const int g_shift = __builtin_ctz((unsigned)a.g);
  auto scale_of = [&](int c) { return g_pow2 ? (c * 32) >> g_shift : (c * 32) / a.g; };
  // lane s < nslots holds slot s's page-table row (down segment), router weight and, when
  // pages hold whole row groups, the address of the page holding this wave's rows: the loop
  // then reads no page table (a scalar table read per batch would delay every batch's loads
  // by its latency)
  const bool group_pages = a.rpp % R == 0;
  // With the gate/up kernel's list of page addresses, whole row groups per page and few slots,
  // the page addresses come through scalar loads (one round trip, no ids), which leaves the
  // vector memory counter to the activations: those go out first, and waiting for the
  // addresses does not wait for them.
  const bool scalar_pages =
      VIB3_DOWN_SCALAR_PAGES && a.bases && group_pages && ns <= kDownScalarSlots;
  const int r0 = min(R * g0, a.M - 1);
  const int page0 = (int)(((uint64_t)(uint32_t)r0 * a.magic) >> 32);  // page of this wave's rows
  uint64_t my_t = 0, my_base = 0;
  float my_w = 1.0f;
  if (lane < ns) {
    if (lane < top_k) my_w = a.wts[lane];
    else if (a.shared_w) my_w = a.shared_w[lane - top_k];  // sigmoid gate of a shared expert
  }
  if (!scalar_pages && lane < ns) {
    const uint64_t* t =
        lane < top_k ? a.routed_table + ((size_t)a.ids[lane] * 3 + 2) * a.max_pages
                     : a.shared_table + ((size_t)(lane - top_k) * 3 + 2) * a.max_pages;
    my_t = (uint64_t)(uintptr_t)t;
    if (group_pages) {
      typedef __attribute__((address_space(1))) const uint64_t gtab;
      my_base = *(gtab*)(t + page0);
    }
  }
  auto scalar_bases = [&]() {  // page addresses from the list the gate/up kernel wrote
    uint64_t bs[kDownScalarSlots];
#pragma unroll
    for (int s = 0; s < kDownScalarSlots; s++)  // slots past the last repeat it
      bs[s] = ld_table(a.bases + (size_t)min(s, ns - 1) * a.bases_stride + page0);
    __builtin_amdgcn_sched_barrier(0);  // (all loads issued before the first wait)
    uint64_t base = 0;
#pragma unroll
    for (int s = 0; s < kDownScalarSlots; s++) base = lane == s ? bs[s] : base;
    return base;
  };

  // one row group per wave (the launcher sizes the grid so); its batches are (slot, pass),
  // passes innermost
  const int n = g0 < G ? ns * P : 0;
  struct Pos { int s, p; };
  auto advance = [&](Pos q) {
    if (++q.p == P) {
      q.p = 0;
      q.s = min(q.s + 1, ns - 1);
    }
    return q;
  };
  auto rl64 = [&](uint64_t v, int l) {
    return ((uint64_t)(uint32_t)__builtin_amdgcn_readlane((int)(v >> 32), l) << 32) |
           (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)v, l);
  };
  // start() runs unconditionally; a batch past the end reads the intermediate (cached in
  // L2) instead of weights. Lanes past the last chunk re-read it (their x is taken as zero).
  auto start = [&](DownRowsBatch<J>& b, Pos q, bool past) {
    const uint8_t* d = nullptr;
    const uint16_t* sc = nullptr;
    if (group_pages) {  // every lane its own row of the group's page
      const uint64_t pb = rl64(my_base, q.s);
      past = past || pb == 0;  // (no address: a down stage launched before any gate/up stage)
      page_row((const uint8_t*)(uintptr_t)pb, min(R * g0 + grp, a.M - 1), a.rpp, a.M, a.magic,
               pk, ng, d, sc);
    } else {
      const MatRef m{(const uint64_t*)(uintptr_t)rl64(my_t, q.s), nullptr, nullptr, a.rpp, a.M,
                     a.magic};
#pragma unroll
      for (int r = 0; r < R; r++) {  // the rows are wave-uniform: scalar table reads
        const uint8_t* dq;
        const uint16_t* sq;
        mat_row<true>(m, min(R * g0 + r, a.M - 1), pk, ng, dq, sq);
        if (grp == r) { d = dq; sc = sq; }
      }
    }
    if (past) {
      d = (const uint8_t*)a.h;
      sc = (const uint16_t*)a.h;
    }
#pragma unroll
    for (int j = 0; j < J; j++) {
      const int c = min(q.p * CPP + sub + L * j, cpr - 1);
      b.w[j] = ld_stream(d + (uint32_t)c * 16u);
      b.q[j] = ld_u16(sc + scale_of(c));
    }
    __builtin_amdgcn_sched_barrier(0);
  };
  float o = 0.0f, acc = 0.0f;
  auto finish = [&](const DownRowsBatch<J>& b, Pos q, bool keep) {
#pragma unroll
    for (int j = 0; j < J; j++) {
      const int c0 = q.p * CPP + sub + L * j;
      const int c = ONE ? c0 : min(c0, cpr - 1);
      const uint4* xp = xq + (size_t)q.s * 4 * CT + c;
      XChunk x;
      const uint4 va = xp[0], vb = xp[CT], vc = xp[2 * CT], vd = xp[3 * CT];
      x.a[0] = as_h2(va.x); x.a[1] = as_h2(va.y); x.a[2] = as_h2(va.z); x.a[3] = as_h2(va.w);
      x.b[0] = as_h2(vb.x); x.b[1] = as_h2(vb.y); x.b[2] = as_h2(vb.z); x.b[3] = as_h2(vb.w);
      x.c[0] = as_h2(vc.x); x.c[1] = as_h2(vc.y); x.c[2] = as_h2(vc.z); x.c[3] = as_h2(vc.w);
      x.d[0] = as_h2(vd.x); x.d[1] = as_h2(vd.y); x.d[2] = as_h2(vd.z); x.d[3] = as_h2(vd.w);
      x.xs8 = xsum[q.s * CT + c];
      const float t = __builtin_fmaf(chunk_dot(b.w[j], x), decode_scale(b.q[j], a.sdt), acc);
      acc = (ONE || c0 < cpr) ? t : acc;  // one pass: x is zero past cpr
    }
    if (q.p == P - 1) {  // the slot's last pass: its row sums, rounded, into the combine
      float dsum = lanes_sum<L>(acc) * kTwo24;
      if (a.round_f16) dsum = (float)(half_t)dsum;
      const float w = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(my_w), q.s));
      const float next = add_mul_rn(o, w, dsum);  // weighted_accumulate_f32 in slot order
      o = keep ? next : o;                         // (engine.rs:5262-5302)
      acc = 0.0f;
    }
  };

  // NB load buffers in a ring: while batch i is reduced, batch i+1 is loading
  DownRowsBatch<J> buf[NB];
  Pos pos[NB];
  pos[0] = Pos{0, 0};
#pragma unroll
  for (int b = 1; b < NB; b++) pos[b] = advance(pos[b - 1]);
  VIB3_TRACE_POINT(1);
  // stage the activations: each thread takes up to three chunks per pass and issues all of
  // their loads before converting any (one round trip per pass, not one per chunk)
  const char* hb = (const char*)a.h;
  const int nitem = ns * CT, bd = (int)blockDim.x;
  auto load_raw = [&](int i0, uint4 (&raw)[3][4]) {
#pragma unroll
    for (int u = 0; u < 3; u++) {
      const int i = min(i0 + u * bd, nitem - 1);
      const int sl = i / CT, c = min(i - sl * CT, cpr - 1);
      const uint4* src = (const uint4*)(hb + ((size_t)sl * a.K + (size_t)c * 32) * 2);
#pragma unroll
      for (int q = 0; q < 4; q++) raw[u][q] = src[q];
    }
  };
  auto stage = [&](int i0, const uint4 (&raw)[3][4]) {
    // Every lane takes delivery of its raw words here, outside the lane-masked region below:
    // a wait inside a region that the wave can skip would leave the compiler unsure whether
    // these loads are done, and it would then wait for every load in flight in the main loop.
#pragma unroll
    for (int u = 0; u < 3; u++)
#pragma unroll
      for (int q = 0; q < 4; q++)
        asm volatile("" ::"v"(raw[u][q].x), "v"(raw[u][q].y), "v"(raw[u][q].z), "v"(raw[u][q].w));
#pragma unroll
    for (int u = 0; u < 3; u++) {
      const int i = i0 + u * bd;
      if (i >= nitem) break;
      const int sl = i / CT, c = i - sl * CT;
      // f16 intermediates are already f16 pairs: the pair layout is a permutation of the
      // words ((x0,x4) (x1,x5) (x2,x6) (x3,x7) of each 8), and the offset term the sum of
      // the 32 values in index order (make_chunk's numbers exactly, without its conversions)
      uint32_t A[4], B[4], C[4], D[4];
      float sum = 0.0f;
#pragma unroll
      for (int q = 0; q < 4; q++) {
        const uint32_t w[4] = {raw[u][q].x, raw[u][q].y, raw[u][q].z, raw[u][q].w};
        A[q] = (w[0] & 0xffffu) | (w[2] << 16);
        B[q] = (w[0] >> 16) | (w[2] & 0xffff0000u);
        C[q] = (w[1] & 0xffffu) | (w[3] << 16);
        D[q] = (w[1] >> 16) | (w[3] & 0xffff0000u);
#pragma unroll
        for (int j = 0; j < 4; j++) {
          sum += f16_to_f32((uint16_t)(w[j] & 0xffff));
          sum += f16_to_f32((uint16_t)(w[j] >> 16));
        }
      }
      const bool in = c < cpr;  // (selected word by word: a select of whole vectors went
                                // through scratch memory)
      auto word4 = [&](const uint32_t (&v)[4]) {
        return make_uint4(in ? v[0] : 0u, in ? v[1] : 0u, in ? v[2] : 0u, in ? v[3] : 0u);
      };
      uint4* xp = xq + (size_t)sl * 4 * CT + c;
      xp[0] = word4(A);
      xp[CT] = word4(B);
      xp[2 * CT] = word4(C);
      xp[3 * CT] = word4(D);
      xsum[sl * CT + c] = in ? 8.0f * kTwoM24 * sum : 0.0f;
    }
  };
  {
    // first pass, every thread (indices clamped): the first weight batches go out behind the
    // (cached) activations, so waiting for the activations does not wait for the weights
    uint4 raw[3][4];
    load_raw((int)threadIdx.x, raw);
    if (scalar_pages) {
      __builtin_amdgcn_sched_barrier(0);  // (the activation loads issue first)
      my_base = scalar_bases();
    }
    // (also for a wave with no batches: every position is valid, and a branch here would make
    // the waits below count for both cases, i.e. wait for the weights too)
#pragma unroll
    for (int b = 0; b + 1 < NB; b++) start(buf[b], pos[b], false);  // rows clamp to M - 1
#ifdef VIB3_TRACE
    VIB3_TRACE_POINT(7);  // first batches issued
#pragma unroll
    for (int u = 0; u < 3; u++)
#pragma unroll
      for (int q = 0; q < 4; q++)
        asm volatile("" ::"v"(raw[u][q].x), "v"(raw[u][q].y), "v"(raw[u][q].z), "v"(raw[u][q].w));
    VIB3_TRACE_POINT(6);  // activations arrived
#endif
    stage((int)threadIdx.x, raw);
  }
  for (int i0 = (int)threadIdx.x + 3 * bd; i0 < nitem; i0 += 3 * bd) {
    uint4 raw[3][4];
    load_raw(i0, raw);
    stage(i0, raw);
  }
  __syncthreads();
  VIB3_TRACE_POINT(2);
  if (n == 0) return;
  // The loop always runs whole rounds of NB batches, and a batch past the end is reduced like
  // the others and then dropped (a select, not a branch): an exit between two batches would
  // give the loop head a path on which a buffer is still loading, and the compiler would then
  // wait there for every load in flight.
  for (int k = 0; k < n; k += NB) {
#pragma unroll
    for (int b = 0; b < NB; b++) {
      // refill the buffer consumed last with batch k + b + NB - 1
      const int nb = (b + NB - 1) % NB;
      pos[nb] = advance(pos[(nb + NB - 1) % NB]);
      // (the explicit wait: see k_int4_rows; here it keeps the compiler's count exact with
      // the past-the-end batches, which read the cached intermediate instead of weights)
      // (batch b's loads done: at most the NB - 2 batches issued after it still loading)
      VIB3_WAIT_VM((NB - 2) * 2 * J);
      start(buf[nb], pos[nb], k + b + NB - 1 >= n);
      finish(buf[b], pos[b], k + b < n);
#ifdef VIB3_TRACE
      if (k + b == 0) VIB3_TRACE_POINT(4);  // first batch reduced
#endif
    }
  }
  VIB3_TRACE_POINT(5);
  // stored after the loop: a store inside it would share the load counter with the weight
  // loads, and the compiler then waits for all of them at the loop head
  const int r = R * g0 + grp;
  if (sub == 0 && r < a.M) a.out[r] = a.residual ? a.residual[r] + o : o;  // engine.rs:5302
  advance_router_tag(a.gen_word);
  VIB3_TRACE_POINT(3);
}

// ------------------------------------------------------------------------- k_int4_generic

template <bool DUAL>
__global__ __launch_bounds__(256) void k_int4_generic(GenericArgs a) {
  const int lane = lane_id();
  const int row = (int)blockIdx.x * 4 + (int)(threadIdx.x >> 6);
  if (row >= a.M) return;
  const int pk = (a.K + 1) / 2, ng = (a.K + a.g - 1) / a.g;
  const uint8_t* d0 = a.data0 + (size_t)row * pk;
  const uint16_t* s0 = a.scales0 + (size_t)row * ng;
  const uint8_t* d1 = DUAL ? a.data1 + (size_t)row * pk : nullptr;
  const uint16_t* s1 = DUAL ? a.scales1 + (size_t)row * ng : nullptr;
  float acc0 = 0.f, acc1 = 0.f;
  for (int col = lane; col < a.K; col += kWave) {
    const float xv = load_act(a.x, a.x_dt, col);
    const int gi = col / a.g;
    uint16_t sb0;
    __builtin_memcpy(&sb0, (const uint8_t*)s0 + 2 * (size_t)gi, 2);
    const uint8_t b0 = d0[col >> 1];
    const int q0 = (col & 1) ? (b0 >> 4) : (b0 & 15);
    acc0 = __builtin_fmaf(xv, (float)(q0 - 8) * decode_scale(sb0, a.sdt), acc0);
    if (DUAL) {
      uint16_t sb1;
      __builtin_memcpy(&sb1, (const uint8_t*)s1 + 2 * (size_t)gi, 2);
      const uint8_t b1 = d1[col >> 1];
      const int q1 = (col & 1) ? (b1 >> 4) : (b1 & 15);
      acc1 = __builtin_fmaf(xv, (float)(q1 - 8) * decode_scale(sb1, a.sdt), acc1);
    }
  }
  const float t0 = wave_sum(acc0);
  const float t1 = DUAL ? wave_sum(acc1) : 0.f;
  if (lane == 0) {
    const float v = DUAL ? (t1 / (1.0f + expf(-t1))) * t0 : t0;
    if (a.out_dt == VIB3_DT_F16) ((uint16_t*)a.out)[row] = f32_to_f16_bits(v);
    else ((float*)a.out)[row] = v;
  }
}

// ------------------------------------------------------------------------- host launchers

static int pick_nch(int cpr, int max_ks, int& nch, int& ks) {
  for (int n : {1, 2, 4}) {
    if (cpr <= kWave * n) { nch = n; ks = 1; return 0; }
  }
  nch = 4;
  ks = (cpr + 4 * kWave - 1) / (4 * kWave);
  if (ks == 3) ks = 4;
  return ks <= max_ks ? 0 : VIB3_ERR_UNSUPPORTED;
}

// Launch-shape constants, fixed at build time (profiling builds may set them with -D):
// workgroups per CU of k_int4_rows (streaming reads peak near 32 KB in flight per CU, not at
// full occupancy), of k_down_combine (0: resident capacity), waves per k_down_rows workgroup
// (0: from the row count), and k_down_combine instead of k_down_rows (1).
#ifndef VIB3_ROWS_BLOCKS_PER_CU
#define VIB3_ROWS_BLOCKS_PER_CU 2
#endif
#ifndef VIB3_DOWN_BLOCKS_PER_CU
#define VIB3_DOWN_BLOCKS_PER_CU 0
#endif
#ifndef VIB3_DOWN_WAVES
#define VIB3_DOWN_WAVES 0
#endif
#ifndef VIB3_DOWN_COMBINE
#define VIB3_DOWN_COMBINE 0
#endif
static int knob(int v, int dflt) { return v > 0 ? v : dflt; }

template <int N, bool D, int S, bool P>
static int rows_grid(const RowsArgs& a) {  // workgroups of a k_int4_rows launch
  auto k = k_int4_rows<N, D, S, P>;
  const int items = a.nslots * a.M;
  const int want = (items + 3) / 4;
  int cap = resident_blocks(k, 256);
  // At most two workgroups per CU: with a third, the CU serves the youngest last and it ends
  // the launch alone (c1: gate/up 26.4 -> 25.0 us with two)
  const int per_cu = knob(VIB3_ROWS_BLOCKS_PER_CU, 2);
  if (per_cu * device_cus() < cap) cap = per_cu * device_cus();
  const int floor_blocks = (items + 4 * kWave - 1) / (4 * kWave);  // <= 64 items per wave
  if (cap < floor_blocks) cap = floor_blocks;
  return want < cap ? want : cap;
}

template <int N, bool D, int S, bool P>
static void launch_rows_p(RowsArgs& a, hipStream_t s, KTime t) {
  if (S == kXi16n || a.KS == 1) {
    const int grid = rows_grid<N, D, S, P>(a);
    if (a.pre_shared) {  // shared items before the selection: only where every wave keeps
      // its items within the 64 lanes that hold them, and for f16 / bf16 activations (with
      // the f32 stream the streaming waves slow the selecting wave more than they gain:
      // sublayer 57.4-57.6 -> 57.7-57.9 us, against 53.7-54.0 -> 52.3-53.2 us for c2)
      const int NP = grid * 3;
      const int Sh = (a.nslots - a.top_k) * a.M, R = a.top_k * a.M, W = 4 * grid;
      a.pre_shared = P && S == kXf16 && a.route == kRouteFused && Sh > 0 && NP > 0 &&
                     (Sh + NP - 1) / NP + (R + W - 1) / W <= kWave;
    }
    hipExtLaunchKernelGGL((k_int4_rows<N, D, S, P>), dim3((unsigned)grid), dim3(256), 0, s,
                          t.start, t.stop, 0, a);
  } else if constexpr (S != kXi16n) {
    a.pre_shared = 0;
    auto k = k_int4_rows_ksplit<N, D, S, P>;
    const int teams = 4 / a.KS;
    dim3 grid((unsigned)((a.M + teams * a.RPT - 1) / (teams * a.RPT)), (unsigned)a.nslots);
    hipExtLaunchKernelGGL(k, grid, dim3(256), 0, s, t.start, t.stop, 0, a);
  }
}


template <int N, bool D, int S>
static void launch_rows_t(RowsArgs& a, hipStream_t s, KTime t) {
  if (S == kXi16n) return launch_rows_p<N, D, kXi16n, true>(a, s, t);  // paged launches only
  if (S == kXi16) return launch_rows_p<N, D, kXi16, true>(a, s, t);
  if (!a.routed_table) return launch_rows_p<N, D, S, false>(a, s, t);
  return launch_rows_p<N, D, S, true>(a, s, t);
}
bool rows_write_bases(const RowsArgs& a) {  // k_int4_rows (one k pass, paged) writes them
  int nch = 1, ks = 1;
  return a.routed_table && a.M > 0 && a.nslots > 0 && !pick_nch(a.K / 32, 4, nch, ks) && ks == 1;
}

// The fused prologue needs the int16 mode of a paged one-pass launch with fused routing, every
// router row in the kernel's split form on a workgroup of its own, and K <= 256 * kNormMax.
bool rows_fuse_prologue(const RowsArgs& a) {
  int nch = 1, ks = 1;
  if (!a.norm_w || a.x_dt != VIB3_DT_F32 || !a.x_i16 || !rows_write_bases(a) ||
      a.route != kRouteFused || a.K > 256 * kNormMax || (a.ngate > 0 && !a.gate_w) ||
      a.ngate > a.router.E)
    return false;
  const RouterArgs& r = a.router;
  if (r.D != a.K || r.D % 8 || r.D / 8 > 4 * 256 || ((uintptr_t)r.w & 15) || ((uintptr_t)a.x & 15) ||
      ((uintptr_t)a.norm_w & 15) || r.x != a.x)
    return false;
  pick_nch(a.K / 32, 4, nch, ks);
  const int grid = nch == 1   ? rows_grid<1, true, kXi16n, true>(a)
                   : nch == 2 ? rows_grid<2, true, kXi16n, true>(a)
                              : rows_grid<4, true, kXi16n, true>(a);
  return r.E <= grid;
}

int launch_rows(RowsArgs a, bool dual, hipStream_t s, KTime t) {
  const int cpr = a.K / 32;
  int nch = 1, ks = 1;
  if (pick_nch(cpr, 4, nch, ks)) return VIB3_ERR_UNSUPPORTED;
  a.KS = ks;
  if (!rows_write_bases(a)) a.down_bases = nullptr;
  if (a.RPT <= 0 || a.RPT > kWave) a.RPT = 8;
  if (a.M <= 0 || a.nslots <= 0) return 0;
  // f32 activations: int16 block fixed point where the caller asks for it (paged layer
  // launches with k in one pass), else the hi + lo f16 split
  int xm = a.x_dt != VIB3_DT_F32 ? kXf16
           : (a.x_i16 && a.routed_table && ks == 1) ? kXi16 : kXsplit;
  if (a.norm_w) {  // a fused prologue asked for: the only mode that applies the norm
    if (!dual || !rows_fuse_prologue(a)) return VIB3_ERR_UNSUPPORTED;
    xm = kXi16n;
  }
#define VIB3_ROWS(N, D)                                   \
  do {                                                    \
    if (D && xm == kXi16n) launch_rows_t<N, true, kXi16n>(a, s, t); \
    else if (xm == kXi16) launch_rows_t<N, D, kXi16>(a, s, t); \
    else if (xm == kXsplit) launch_rows_t<N, D, kXsplit>(a, s, t); \
    else launch_rows_t<N, D, kXf16>(a, s, t);             \
  } while (0)
  if (dual) {
    if (nch == 1) VIB3_ROWS(1, true);
    else if (nch == 2) VIB3_ROWS(2, true);
    else VIB3_ROWS(4, true);
  } else {
    if (nch == 1) VIB3_ROWS(1, false);
    else if (nch == 2) VIB3_ROWS(2, false);
    else VIB3_ROWS(4, false);
  }
#undef VIB3_ROWS
  VIB3_RETURN_LAUNCH();
}

template <bool S, bool W>
static void launch_down_t(DownArgs& a, hipStream_t s, KTime t) {
  auto k = k_down_combine<S, W>;
  const int block = a.nslots * a.KS * kWave;
  int cap = resident_blocks(k, block);
  const int per_cu = knob(VIB3_DOWN_BLOCKS_PER_CU, 0);
  if (per_cu > 0 && per_cu * device_cus() < cap) cap = per_cu * device_cus();
  // rows per block: spread the rows evenly over the resident workgroups, a multiple of the
  // 8-row batch, at most 64 (one LDS column per row)
  int rb = (a.M + cap - 1) / cap;
  rb = (rb + 7) / 8 * 8;  // multiple of both batch heights (4 and 8)
  if (rb > kWave) rb = kWave;
  a.RB = rb;
  const int blocks = (a.M + rb - 1) / rb;
  hipExtLaunchKernelGGL(k, dim3((unsigned)(blocks < cap ? blocks : cap)), dim3((unsigned)block), 0,
                        s, t.start, t.stop, 0, a);
}

#ifndef VIB3_DOWN_ROWS_BUFFERS
#define VIB3_DOWN_ROWS_BUFFERS 2  // load buffers per wave (build-time tuning knob)
#endif
constexpr int kDownRowsBuffers = VIB3_DOWN_ROWS_BUFFERS;

// LDS bytes of k_down_rows: per slot, every chunk's 4 pair words and one offset term.
static size_t down_rows_lds(int nslots, int chunks) {
  return (size_t)nslots * chunks * (64 + 4);
}

template <int R, int J, bool ONE>
static void launch_down_rows_t(DownArgs& a, hipStream_t s, KTime t) {
  // One row group per wave, and as many waves per workgroup as make one workgroup per CU
  // (2..8): every CU streams the same share of the weights, and stages the activations once.
  // (Four-wave workgroups left some CUs two workgroups and others one.)
  const int groups = (a.M + R - 1) / R;
  int wpb = knob(VIB3_DOWN_WAVES, (groups + device_cus() - 1) / device_cus());
  wpb = wpb < 2 ? 2 : wpb > 8 ? 8 : wpb;
  const int blocks = (groups + wpb - 1) / wpb;
  const int chunks = ONE ? kWave / R * J : a.K / 32;
  hipExtLaunchKernelGGL((k_down_rows<R, J, kDownRowsBuffers, ONE>), dim3((unsigned)blocks),
                        dim3(64 * wpb), (unsigned)down_rows_lds(a.nslots, chunks), s, t.start,
                        t.stop, 0, a);
}

template <int R>
static void launch_down_rows_j(DownArgs& a, int cpr, hipStream_t s, KTime t) {
  constexpr int L = kWave / R;  // J: chunks per lane per pass, enough for one pass up to 4
  if (cpr <= L) launch_down_rows_t<R, 1, true>(a, s, t);
  else if (cpr <= 2 * L) launch_down_rows_t<R, 2, true>(a, s, t);
  else if (cpr <= 4 * L) launch_down_rows_t<R, 4, true>(a, s, t);
  else launch_down_rows_t<R, 4, false>(a, s, t);
}

int launch_down(DownArgs a, hipStream_t s, KTime t) {
  const int cpr = a.K / 32;
  if (a.M <= 0) return 0;
  // staged-activation kernel for f16 intermediates whose staged form fits 64 KB of LDS;
  // rows per wave: 4 while that leaves enough row groups to fill the GPU, else 2 or 1
  const int waves = 6 * device_cus();
  const int R = a.M / 4 >= waves ? 4 : a.M / 2 >= waves ? 2 : 1;
  const int L = kWave / R;  // the LDS holds one pass's chunks (padded) or all cpr
  const int chunks = cpr <= L ? L : cpr <= 2 * L ? 2 * L : cpr <= 4 * L ? 4 * L : cpr;
  if (a.h_dt == VIB3_DT_F16 && down_rows_lds(a.nslots, chunks) <= 64 * 1024 &&
      VIB3_DOWN_COMBINE == 0) {
    if (R == 4) launch_down_rows_j<4>(a, cpr, s, t);
    else if (R == 2) launch_down_rows_j<2>(a, cpr, s, t);
    else launch_down_rows_j<1>(a, cpr, s, t);
    VIB3_RETURN_LAUNCH();
  }
  const int ks = (cpr + kDownSpan - 1) / kDownSpan;
  if (a.nslots * ks > 16) return VIB3_ERR_UNSUPPORTED;
  a.KS = ks;
  if (a.M <= 0) return 0;
  const bool wide = a.nslots * ks > 10;
  if (a.h_dt == VIB3_DT_F32) {
    if (wide) launch_down_t<true, true>(a, s, t);
    else launch_down_t<true, false>(a, s, t);
  } else {
    if (wide) launch_down_t<false, true>(a, s, t);
    else launch_down_t<false, false>(a, s, t);
  }
  VIB3_RETURN_LAUNCH();
}

int launch_generic(GenericArgs a, bool dual, hipStream_t s) {
  dim3 grid((unsigned)((a.M + 3) / 4));
  if (grid.x == 0) return 0;
  if (dual) hipLaunchKernelGGL((k_int4_generic<true>), grid, dim3(256), 0, s, a);
  else hipLaunchKernelGGL((k_int4_generic<false>), grid, dim3(256), 0, s, a);
  VIB3_RETURN_LAUNCH();
}

}  // namespace vib3

#ifdef VIB3_TRACE
// Profiling builds only: where this translation unit's kernels write their timeline probes
// (16 u64 per workgroup).
extern "C" int vib3_trace_set(void* buf) {
  uint64_t* p = (uint64_t*)buf;
  return (int)hipMemcpyToSymbol(HIP_SYMBOL(vib3_trace_buf), &p, sizeof(p));
}
#endif
