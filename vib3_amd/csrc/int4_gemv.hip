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

template <int NCH, bool DUAL, int U>
__device__ __forceinline__ void issue(RowBatch<NCH, DUAL, U>& b, const MatRef& m0, const MatRef& m1,
                                      const int (&ra)[U], const int (&cidx)[NCH],
                                      const int (&gidx)[NCH], int pk, int ng, int cpr) {
#pragma unroll
  for (int u = 0; u < U; u++) {
    const uint8_t *d0, *d1 = nullptr;
    const uint16_t *s0, *s1 = nullptr;
    mat_row(m0, ra[u], pk, ng, d0, s0);
    if (DUAL) mat_row(m1, ra[u], pk, ng, d1, s1);
#pragma unroll
    for (int j = 0; j < NCH; j++) {
      // lanes past the last chunk re-read it (no divergent branch around the loads); their
      // activation chunk is zero, so they add nothing
      const int c = min(cidx[j], cpr - 1);
      const size_t off = (size_t)c * 16;
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
template <int NCH, bool DUAL, bool SPLIT, int U>
__device__ __forceinline__ void reduce(const RowBatch<NCH, DUAL, U>& b, const XChunk (&xh)[NCH],
                                       const XChunk (&xl)[NCH], const int (&cidx)[NCH], int cpr,
                                       int sdt, float (&t0)[U], float (&t1)[U]) {
#pragma unroll
  for (int u = 0; u < U; u++) {
    float acc0 = 0.f, acc1 = 0.f;
#pragma unroll
    for (int j = 0; j < NCH; j++) {
      float p0 = chunk_dot(b.w0[u][j], xh[j]);
      if (SPLIT) p0 += chunk_dot(b.w0[u][j], xl[j]);
      acc0 = __builtin_fmaf(p0, decode_scale(b.q0[u][j], sdt), acc0);
      if (DUAL) {
        float p1 = chunk_dot(b.w1[u][j], xh[j]);
        if (SPLIT) p1 += chunk_dot(b.w1[u][j], xl[j]);
        acc1 = __builtin_fmaf(p1, decode_scale(b.q1[u][j], sdt), acc1);
      }
    }
    t0[u] = wave_sum(acc0) * kTwo24;
    t1[u] = DUAL ? wave_sum(acc1) * kTwo24 : 0.f;
  }
}

template <int NCH, bool DUAL, bool SPLIT, int U>
__device__ __forceinline__ void dot_rows(const MatRef& m0, const MatRef& m1, const int (&ra)[U],
                                         const XChunk (&xh)[NCH], const XChunk (&xl)[NCH],
                                         const int (&cidx)[NCH], const int (&gidx)[NCH], int pk,
                                         int ng, int cpr, int sdt, float (&t0)[U], float (&t1)[U]) {
  RowBatch<NCH, DUAL, U> b;
  issue<NCH, DUAL, U>(b, m0, m1, ra, cidx, gidx, pk, ng, cpr);
  reduce<NCH, DUAL, SPLIT, U>(b, xh, xl, cidx, cpr, sdt, t0, t1);
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
template <int NCH, bool SPLIT>
__device__ __forceinline__ void load_x(const void* x, int x_dt, int cpr, const int (&cidx)[NCH],
                                       XChunk (&xh)[NCH], XChunk (&xl)[NCH]) {
#pragma unroll
  for (int j = 0; j < NCH; j++) {
    if (cidx[j] < cpr) {
      float xv[32];
      load_chunk_act(x, x_dt, cidx[j], xv);
      make_chunk(xv, xh[j], xl[j]);
      if (!SPLIT) zero_chunk(xl[j]);
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
  if (!a.routed_table) return which == 0 ? a.flat0 : a.flat1;
  const uint64_t* t;
  if (slot < a.top_k) t = a.routed_table + ((size_t)expert * 3 + seg) * a.max_pages;
  else t = a.shared_table + ((size_t)(slot - a.top_k) * 3 + seg) * a.max_pages;
  return MatRef{t, nullptr, nullptr, a.rpp[seg], a.M};
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

template <int NCH, bool DUAL, bool SPLIT>
__global__ __launch_bounds__(256) void k_int4_rows(RowsArgs a) {
  const int lane = lane_id();
  const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));  // wave-uniform (SGPR)
  const int pk = a.K / 2, ng = (a.K + a.g - 1) / a.g, cpr = a.K / 32;
  XChunk xh[NCH], xl[NCH];
  int cidx[NCH], gidx[NCH];

  if (a.KS == 1) {
    // Items are (slot, row), shared-expert slots first; waves stride over them. Two load
    // buffers alternate so the next item's 16-byte loads are in flight while the current one
    // is reduced (no register copies of in-flight loads, which would force a wait).
    __shared__ int s_sel[64];
    __shared__ float s_wts[64];
    chunk_index<NCH>(0, a.g, cpr, cidx, gidx);
    const int items = a.nslots * a.M;
    const int stride = (int)gridDim.x * 4;
    int it = (int)blockIdx.x * 4 + wave;
    auto slot_of = [&](int item) {
      const int q = item / a.M;
      return a.nslots > a.top_k ? (q + a.top_k) % a.nslots : q;
    };
    auto expert_of = [&](int slot) {
      if (slot >= a.top_k || !a.routed_table) return 0;
      return a.route ? __builtin_amdgcn_readfirstlane(s_sel[slot]) : (int)a.ids[slot];
    };
    RowBatch<NCH, DUAL, 1> A, B;
    auto start = [&](RowBatch<NCH, DUAL, 1>& buf, int item) {
      const int slot = slot_of(item);
      const int e = expert_of(slot);
      const MatRef m0 = slot_matrix(a, slot, e, 0, 0);
      const MatRef m1 = DUAL ? slot_matrix(a, slot, e, 1, 1) : m0;
      const int ra[1] = {item - (item / a.M) * a.M};
      issue<NCH, DUAL, 1>(buf, m0, m1, ra, cidx, gidx, pk, ng, cpr);
    };
    auto finish = [&](const RowBatch<NCH, DUAL, 1>& buf, int item) {
      float t0[1], t1[1];
      reduce<NCH, DUAL, SPLIT, 1>(buf, xh, xl, cidx, cpr, a.sdt, t0, t1);
      const int slot = slot_of(item);
      if (lane == 0)
        store_out(a, (size_t)slot * a.out_stride + (item - (item / a.M) * a.M),
                  rows_epilogue(DUAL, t0[0], t1[0]));
    };
    // a shared-expert row needs no routing: start its loads before the selection
    const bool early = it < items && slot_of(it) >= a.top_k;
    if (early) start(A, it);
    if (a.route) {
      if (wave == 0) select_topk_regs<8>(a.router, a.router.scores, s_sel, s_wts, blockIdx.x == 0);
      __syncthreads();
    }
    if (it >= items) return;
    if (!early) start(A, it);
    load_x<NCH, SPLIT>(a.x, a.x_dt, cpr, cidx, xh, xl);
    for (;;) {
      const int i1 = it + stride;
      if (i1 < items) start(B, i1);
      finish(A, it);
      if (i1 >= items) break;
      const int i2 = i1 + stride;
      if (i2 < items) start(A, i2);
      finish(B, i1);
      if (i2 >= items) break;
      it = i2;
    }
    return;
  }

  const int ks = wave % a.KS;
  const int team = wave / a.KS;
  const int teams = 4 / a.KS;
  const int slot = (int)blockIdx.y;
  const int r0 = ((int)blockIdx.x * teams + team) * a.RPT;
  const int nrows = max(0, min(a.RPT, a.M - r0));
  const int e = (a.routed_table && slot < a.top_k) ? (int)a.ids[slot] : 0;
  const MatRef m0 = slot_matrix(a, slot, e, 0, 0);
  const MatRef m1 = DUAL ? slot_matrix(a, slot, e, 1, 1) : m0;
  chunk_index<NCH>(ks, a.g, cpr, cidx, gidx);
  load_x<NCH, SPLIT>(a.x, a.x_dt, cpr, cidx, xh, xl);
  float res0 = 0.f, res1 = 0.f;
  for (int i = 0; i < nrows; i += 2) {
    const int ra[2] = {r0 + i, i + 1 < nrows ? r0 + i + 1 : r0 + i};
    float t0[2], t1[2];
    dot_rows<NCH, DUAL, SPLIT, 2>(m0, m1, ra, xh, xl, cidx, gidx, pk, ng, cpr, a.sdt, t0, t1);
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
// One workgroup = nslots * KS waves (one wave per expert slot and k part); it strides over
// blocks of RB output rows. Each wave computes its slot's rows, the per-row results meet in
// LDS, and wave 0 forms sum_s w_s * f16(d_s) in slot order (router order, then shared).

template <int NCH, bool SPLIT>
__global__ __launch_bounds__(1024) void k_down_combine(DownArgs a) {
  const int lane = lane_id();
  const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));  // wave-uniform (SGPR)
  const int slot = wave / a.KS;
  const int ks = wave % a.KS;
  const int pk = a.K / 2, ng = (a.K + a.g - 1) / a.g, cpr = a.K / 32;

  const uint64_t* t = slot < a.top_k
                          ? a.routed_table + ((size_t)a.ids[slot] * 3 + 2) * a.max_pages
                          : a.shared_table + ((size_t)(slot - a.top_k) * 3 + 2) * a.max_pages;
  const MatRef m{t, nullptr, nullptr, a.rpp, a.M};
  XChunk xh[NCH], xl[NCH];
  int cidx[NCH], gidx[NCH];
  chunk_index<NCH>(ks, a.g, cpr, cidx, gidx);
  const char* hbase = (const char*)a.h + (size_t)slot * a.K * (a.h_dt == VIB3_DT_F32 ? 4 : 2);

  constexpr int U = NCH == 1 ? 4 : 2;  // rows per batch (keeps NCH=2 within 128 VGPRs)
  // This workgroup's items: blocks b = blockIdx.x + n * gridDim.x, each in ceil(RB / U)
  // batches of U rows (the last block's surplus rows repeat its last row and are dropped).
  // Two load buffers alternate; the first batch is issued before h is even read.
  __shared__ float part[16][kWave];
  const int blocks = (a.M + a.RB - 1) / a.RB;
  if ((int)blockIdx.x >= blocks) return;
  const int ipb = (a.RB + U - 1) / U;
  const int my_blocks = (blocks - (int)blockIdx.x + (int)gridDim.x - 1) / (int)gridDim.x;
  const int n = my_blocks * ipb;
  RowBatch<NCH, false, U> A, B;
  float res = 0.f;
  auto start = [&](RowBatch<NCH, false, U>& buf, int k) {
    const int bb = (int)blockIdx.x + (k / ipb) * (int)gridDim.x;
    const int r0 = bb * a.RB, nr = min(a.RB, a.M - r0), i0 = (k % ipb) * U;
    int ra[U];
#pragma unroll
    for (int u = 0; u < U; u++) ra[u] = r0 + min(i0 + u, nr - 1);
    issue<NCH, false, U>(buf, m, m, ra, cidx, gidx, pk, ng, cpr);
  };
  auto finish = [&](const RowBatch<NCH, false, U>& buf, int k) {
    const int bb = (int)blockIdx.x + (k / ipb) * (int)gridDim.x;
    const int r0 = bb * a.RB, nr = min(a.RB, a.M - r0), i0 = (k % ipb) * U;
    float t0[U], t1[U];
    reduce<NCH, false, SPLIT, U>(buf, xh, xl, cidx, cpr, a.sdt, t0, t1);
#pragma unroll
    for (int u = 0; u < U; u++)
      if (lane == i0 + u) res = t0[u];
    if (k % ipb == ipb - 1) {
      // block complete: combine the slots' rows
      part[wave][lane] = res;
      __syncthreads();
      if (wave == 0 && lane < nr) {
        // weighted_accumulate_f32 over the slots in router order, then the shared experts
        // with weight 1.0 (engine.rs:5262-5302): o = o + w * d with separate roundings.
        float o = 0.0f;
        for (int s = 0; s < a.nslots; s++) {
          float d = 0.0f;
          for (int q = 0; q < a.KS; q++) d += part[s * a.KS + q][lane];
          if (a.round_f16) d = (float)(half_t)d;
          const float w = s < a.top_k ? a.wts[s] : 1.0f;
          o = add_mul_rn(o, w, d);
        }
        a.out[r0 + lane] = o;
      }
      __syncthreads();
      res = 0.f;
    }
  };
  start(A, 0);
  load_x<NCH, SPLIT>(hbase, a.h_dt, cpr, cidx, xh, xl);
  for (int k = 0;; k += 2) {
    if (k + 1 < n) start(B, k + 1);
    finish(A, k);
    if (k + 1 >= n) break;
    if (k + 2 < n) start(A, k + 2);
    finish(B, k + 1);
    if (k + 2 >= n) break;
  }
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

// Resident workgroups per CU for a kernel at a block size, and the CU count (cached per device;
// plain host queries, no allocation).
static int device_cus() {
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
static int resident_blocks(K kernel, int block) {
  int per_cu = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kernel, block, 0) != hipSuccess ||
      per_cu <= 0)
    per_cu = 1;
  return per_cu * device_cus();
}

static int pick_nch(int cpr, int max_ks, int& nch, int& ks) {
  for (int n : {1, 2, 4}) {
    if (cpr <= kWave * n) { nch = n; ks = 1; return 0; }
  }
  nch = 4;
  ks = (cpr + 4 * kWave - 1) / (4 * kWave);
  if (ks == 3) ks = 4;
  return ks <= max_ks ? 0 : VIB3_ERR_UNSUPPORTED;
}

// Resident-capacity cap on the number of 256-thread blocks; VIB3_ROWS_BLOCKS_PER_CU overrides
// (tuning knob; streaming reads peak near 32 KB in flight per CU, not at full occupancy).
static int env_int(const char* name, int dflt) {
  const char* v = getenv(name);
  return v && atoi(v) > 0 ? atoi(v) : dflt;
}

template <int N, bool D, bool S>
static void launch_rows_t(RowsArgs& a, hipStream_t s) {
  auto k = k_int4_rows<N, D, S>;
  if (a.KS == 1) {
    const int items = a.nslots * a.M;
    const int want = (items + 3) / 4;
    int cap = resident_blocks(k, 256);
    const int per_cu = env_int("VIB3_ROWS_BLOCKS_PER_CU", 0);
    if (per_cu > 0 && per_cu * device_cus() < cap) cap = per_cu * device_cus();
    hipLaunchKernelGGL(k, dim3((unsigned)(want < cap ? want : cap)), dim3(256), 0, s, a);
  } else {
    const int teams = 4 / a.KS;
    dim3 grid((unsigned)((a.M + teams * a.RPT - 1) / (teams * a.RPT)), (unsigned)a.nslots);
    hipLaunchKernelGGL(k, grid, dim3(256), 0, s, a);
  }
}

int launch_rows(RowsArgs a, bool dual, hipStream_t s) {
  const int cpr = a.K / 32;
  int nch = 1, ks = 1;
  if (pick_nch(cpr, 4, nch, ks)) return VIB3_ERR_UNSUPPORTED;
  a.KS = ks;
  if (a.RPT <= 0 || a.RPT > kWave) a.RPT = 8;
  if (a.M <= 0 || a.nslots <= 0) return 0;
  const bool split = a.x_dt == VIB3_DT_F32;
#define VIB3_ROWS(N, D)                                   \
  do {                                                    \
    if (split) launch_rows_t<N, D, true>(a, s);           \
    else launch_rows_t<N, D, false>(a, s);                \
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

template <int N, bool S>
static void launch_down_t(DownArgs& a, hipStream_t s) {
  auto k = k_down_combine<N, S>;
  const int block = a.nslots * a.KS * kWave;
  int cap = resident_blocks(k, block);
  const int per_cu = env_int("VIB3_DOWN_BLOCKS_PER_CU", 0);
  if (per_cu > 0 && per_cu * device_cus() < cap) cap = per_cu * device_cus();
  // rows per block: spread the rows evenly over the resident workgroups, multiple of 4
  int rb = (a.M + cap - 1) / cap;
  rb = (rb + 3) / 4 * 4;  // a multiple of both batch sizes (4 and 2)
  if (rb > kWave) rb = kWave;
  a.RB = rb;
  const int blocks = (a.M + rb - 1) / rb;
  hipLaunchKernelGGL(k, dim3((unsigned)(blocks < cap ? blocks : cap)), dim3((unsigned)block), 0,
                     s, a);
}

int launch_down(DownArgs a, hipStream_t s) {
  const int cpr = a.K / 32;
  // NCH <= 2 keeps a 1024-thread workgroup within 128 VGPRs per lane.
  const int nch = cpr <= kWave ? 1 : 2;
  const int ks = (cpr + nch * kWave - 1) / (nch * kWave);
  if (a.nslots * ks > 16) return VIB3_ERR_UNSUPPORTED;
  a.KS = ks;
  if (a.M <= 0) return 0;
  const bool split = a.h_dt == VIB3_DT_F32;
  if (nch == 1) {
    if (split) launch_down_t<1, true>(a, s);
    else launch_down_t<1, false>(a, s);
  } else {
    if (split) launch_down_t<2, true>(a, s);
    else launch_down_t<2, false>(a, s);
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
