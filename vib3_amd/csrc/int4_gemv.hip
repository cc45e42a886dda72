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
#include "common.h"
#include "kernels.h"

namespace vib3 {

// ------------------------------------------------------------------------- k_int4_rows

template <int NCH, bool DUAL, bool SPLIT>
__device__ __forceinline__ void rows_loop(const RowsArgs& a, const MatRef& m0, const MatRef& m1,
                                          const XChunk (&xh)[NCH], const XChunk (&xl)[NCH],
                                          const int (&cidx)[NCH], const int (&gidx)[NCH],
                                          int r0, int nrows, int pk, int ng, int cpr,
                                          float& res0, float& res1) {
  const int lane = lane_id();
  for (int i = 0; i < nrows; i += 2) {
    const int ra = r0 + i;
    const bool vb = i + 1 < nrows;
    const int rb = vb ? ra + 1 : ra;
    const uint8_t *d0a, *d0b, *d1a = nullptr, *d1b = nullptr;
    const uint16_t *s0a, *s0b, *s1a = nullptr, *s1b = nullptr;
    mat_row(m0, ra, pk, ng, d0a, s0a);
    mat_row(m0, rb, pk, ng, d0b, s0b);
    if (DUAL) {
      mat_row(m1, ra, pk, ng, d1a, s1a);
      mat_row(m1, rb, pk, ng, d1b, s1b);
    }
    uint4 w0a[NCH], w0b[NCH], w1a[NCH], w1b[NCH];
    uint16_t q0a[NCH], q0b[NCH], q1a[NCH], q1b[NCH];
#pragma unroll
    for (int j = 0; j < NCH; j++) {
      if (cidx[j] < cpr) {
        const size_t off = (size_t)cidx[j] * 16;
        w0a[j] = ld_stream(d0a + off);
        w0b[j] = ld_stream(d0b + off);
        q0a[j] = s0a[gidx[j]];
        q0b[j] = s0b[gidx[j]];
        if (DUAL) {
          w1a[j] = ld_stream(d1a + off);
          w1b[j] = ld_stream(d1b + off);
          q1a[j] = s1a[gidx[j]];
          q1b[j] = s1b[gidx[j]];
        }
      }
    }
    float acc0a = 0.f, acc0b = 0.f, acc1a = 0.f, acc1b = 0.f;
#pragma unroll
    for (int j = 0; j < NCH; j++) {
      if (cidx[j] < cpr) {
        float p0a = chunk_dot(w0a[j], xh[j]);
        float p0b = chunk_dot(w0b[j], xh[j]);
        if (SPLIT) {
          p0a += chunk_dot(w0a[j], xl[j]);
          p0b += chunk_dot(w0b[j], xl[j]);
        }
        acc0a = __builtin_fmaf(p0a, decode_scale(q0a[j], a.sdt), acc0a);
        acc0b = __builtin_fmaf(p0b, decode_scale(q0b[j], a.sdt), acc0b);
        if (DUAL) {
          float p1a = chunk_dot(w1a[j], xh[j]);
          float p1b = chunk_dot(w1b[j], xh[j]);
          if (SPLIT) {
            p1a += chunk_dot(w1a[j], xl[j]);
            p1b += chunk_dot(w1b[j], xl[j]);
          }
          acc1a = __builtin_fmaf(p1a, decode_scale(q1a[j], a.sdt), acc1a);
          acc1b = __builtin_fmaf(p1b, decode_scale(q1b[j], a.sdt), acc1b);
        }
      }
    }
    const float t0a = wave_sum(acc0a) * kTwo24;
    const float t0b = wave_sum(acc0b) * kTwo24;
    if (lane == i) res0 = t0a;
    if (lane == i + 1) res0 = t0b;
    if (DUAL) {
      const float t1a = wave_sum(acc1a) * kTwo24;
      const float t1b = wave_sum(acc1b) * kTwo24;
      if (lane == i) res1 = t1a;
      if (lane == i + 1) res1 = t1b;
    }
  }
}

__device__ __forceinline__ MatRef slot_matrix(const RowsArgs& a, int slot, int seg, int which) {
  if (!a.routed_table) return which == 0 ? a.flat0 : a.flat1;
  const uint64_t* t;
  if (slot < a.top_k) t = a.routed_table + ((size_t)a.ids[slot] * 3 + seg) * a.max_pages;
  else t = a.shared_table + ((size_t)(slot - a.top_k) * 3 + seg) * a.max_pages;
  return MatRef{t, nullptr, nullptr, a.rpp[seg], a.M};
}

template <int NCH, bool DUAL>
__global__ __launch_bounds__(256) void k_int4_rows(RowsArgs a) {
  const int lane = lane_id();
  const int wave = (int)(threadIdx.x >> 6);
  const int ks = wave % a.KS;
  const int team = wave / a.KS;
  const int teams = 4 / a.KS;
  const int slot = (int)blockIdx.y;
  const int r0 = ((int)blockIdx.x * teams + team) * a.RPT;
  const int nrows = max(0, min(a.RPT, a.M - r0));
  const int pk = a.K / 2, ng = (a.K + a.g - 1) / a.g, cpr = a.K / 32;

  const MatRef m0 = slot_matrix(a, slot, 0, 0);
  const MatRef m1 = DUAL ? slot_matrix(a, slot, 1, 1) : m0;

  XChunk xh[NCH], xl[NCH];
  int cidx[NCH], gidx[NCH];
  bool need = false;
#pragma unroll
  for (int j = 0; j < NCH; j++) {
    cidx[j] = (ks * NCH + j) * kWave + lane;
    gidx[j] = (cidx[j] * 32) / a.g;
    if (cidx[j] < cpr) {
      float xv[32];
      load_chunk_act(a.x, a.x_dt, cidx[j], xv);
      need |= make_chunk(xv, xh[j], xl[j]);
    } else {
      zero_chunk(xh[j]);
      zero_chunk(xl[j]);
    }
  }
  const bool split = __any((int)need);

  float res0 = 0.f, res1 = 0.f;
  if (nrows > 0) {
    if (split)
      rows_loop<NCH, DUAL, true>(a, m0, m1, xh, xl, cidx, gidx, r0, nrows, pk, ng, cpr, res0, res1);
    else
      rows_loop<NCH, DUAL, false>(a, m0, m1, xh, xl, cidx, gidx, r0, nrows, pk, ng, cpr, res0, res1);
  }

  if (a.KS > 1) {
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
  }
  if (lane < nrows) {
    // DUAL: matrix 0 = up (segment 0), matrix 1 = gate (segment 1); silu goes on the gate.
    const float v = DUAL ? (res1 / (1.0f + expf(-res1))) * res0 : res0;
    const size_t o = (size_t)slot * a.out_stride + r0 + lane;
    if (a.out_dt == VIB3_DT_F16) ((uint16_t*)a.out)[o] = f32_to_f16_bits(v);
    else ((float*)a.out)[o] = v;
  }
}

// ------------------------------------------------------------------------- k_down_combine

template <int NCH, bool SPLIT>
__device__ __forceinline__ void down_loop(const DownArgs& a, const MatRef& m, const XChunk (&xh)[NCH],
                                          const XChunk (&xl)[NCH], const int (&cidx)[NCH],
                                          const int (&gidx)[NCH], int r0, int nrows, int pk,
                                          int ng, int cpr, float& res) {
  const int lane = lane_id();
  for (int i = 0; i < nrows; i += 2) {
    const int ra = r0 + i;
    const bool vb = i + 1 < nrows;
    const int rb = vb ? ra + 1 : ra;
    const uint8_t *da, *db;
    const uint16_t *sa, *sb;
    mat_row(m, ra, pk, ng, da, sa);
    mat_row(m, rb, pk, ng, db, sb);
    uint4 wa[NCH], wb[NCH];
    uint16_t qa[NCH], qb[NCH];
#pragma unroll
    for (int j = 0; j < NCH; j++) {
      if (cidx[j] < cpr) {
        const size_t off = (size_t)cidx[j] * 16;
        wa[j] = ld_stream(da + off);
        wb[j] = ld_stream(db + off);
        qa[j] = sa[gidx[j]];
        qb[j] = sb[gidx[j]];
      }
    }
    float acca = 0.f, accb = 0.f;
#pragma unroll
    for (int j = 0; j < NCH; j++) {
      if (cidx[j] < cpr) {
        float pa = chunk_dot(wa[j], xh[j]);
        float pb = chunk_dot(wb[j], xh[j]);
        if (SPLIT) {
          pa += chunk_dot(wa[j], xl[j]);
          pb += chunk_dot(wb[j], xl[j]);
        }
        acca = __builtin_fmaf(pa, decode_scale(qa[j], a.sdt), acca);
        accb = __builtin_fmaf(pb, decode_scale(qb[j], a.sdt), accb);
      }
    }
    const float ta = wave_sum(acca) * kTwo24;
    const float tb = wave_sum(accb) * kTwo24;
    if (lane == i) res = ta;
    if (lane == i + 1) res = tb;
  }
}

template <int NCH>
__global__ __launch_bounds__(1024) void k_down_combine(DownArgs a) {
  const int lane = lane_id();
  const int wave = (int)(threadIdx.x >> 6);
  const int slot = wave / a.KS;
  const int ks = wave % a.KS;
  const int r0 = (int)blockIdx.x * a.RB;
  const int nrows = max(0, min(a.RB, a.M - r0));
  const int pk = a.K / 2, ng = (a.K + a.g - 1) / a.g, cpr = a.K / 32;

  const uint64_t* t = slot < a.top_k
                          ? a.routed_table + ((size_t)a.ids[slot] * 3 + 2) * a.max_pages
                          : a.shared_table + ((size_t)(slot - a.top_k) * 3 + 2) * a.max_pages;
  const MatRef m{t, nullptr, nullptr, a.rpp, a.M};

  XChunk xh[NCH], xl[NCH];
  int cidx[NCH], gidx[NCH];
  bool need = false;
  const char* hbase = (const char*)a.h + (size_t)slot * a.K * (a.h_dt == VIB3_DT_F32 ? 4 : 2);
#pragma unroll
  for (int j = 0; j < NCH; j++) {
    cidx[j] = (ks * NCH + j) * kWave + lane;
    gidx[j] = (cidx[j] * 32) / a.g;
    if (cidx[j] < cpr) {
      float xv[32];
      load_chunk_act(hbase, a.h_dt, cidx[j], xv);
      need |= make_chunk(xv, xh[j], xl[j]);
    } else {
      zero_chunk(xh[j]);
      zero_chunk(xl[j]);
    }
  }
  const bool split = __any((int)need);
  float res = 0.f;
  if (nrows > 0) {
    if (split) down_loop<NCH, true>(a, m, xh, xl, cidx, gidx, r0, nrows, pk, ng, cpr, res);
    else down_loop<NCH, false>(a, m, xh, xl, cidx, gidx, r0, nrows, pk, ng, cpr, res);
  }

  __shared__ float part[16][kWave];
  part[wave][lane] = res;
  __syncthreads();
  if (wave != 0 || lane >= nrows) return;
  // weighted_accumulate_f32 over the slots in router order, then the shared experts with
  // weight 1.0 (engine.rs:5262-5302): o = o + w * d with separate roundings, as the reference.
  float o = 0.0f;
  for (int s = 0; s < a.nslots; s++) {
    float d = 0.0f;
    for (int q = 0; q < a.KS; q++) d += part[s * a.KS + q][lane];
    if (a.round_f16) d = (float)(half_t)d;
    const float w = s < a.top_k ? a.wts[s] : 1.0f;
    o = __fadd_rn(o, __fmul_rn(w, d));
  }
  a.out[r0 + lane] = o;
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
    int k = (cpr + kWave * n - 1) / (kWave * n);
    if (k <= 1) { nch = n; ks = 1; return 0; }
  }
  nch = 4;
  ks = (cpr + 4 * kWave - 1) / (4 * kWave);
  if (ks == 3) ks = 4;
  return ks <= max_ks ? 0 : VIB3_ERR_UNSUPPORTED;
}

int launch_rows(RowsArgs a, bool dual, hipStream_t s) {
  const int cpr = a.K / 32;
  int nch = 1, ks = 1;
  if (pick_nch(cpr, 4, nch, ks)) return VIB3_ERR_UNSUPPORTED;
  a.KS = ks;
  if (a.RPT <= 0) a.RPT = 8;
  const int teams = 4 / ks;
  dim3 grid((unsigned)((a.M + teams * a.RPT - 1) / (teams * a.RPT)), (unsigned)a.nslots);
  if (grid.x == 0 || a.nslots == 0) return 0;
#define VIB3_ROWS(N, D) hipLaunchKernelGGL((k_int4_rows<N, D>), grid, dim3(256), 0, s, a)
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

int launch_down(DownArgs a, hipStream_t s) {
  const int cpr = a.K / 32;
  // NCH <= 2 keeps the 1024-thread workgroup within 128 VGPRs per lane.
  int nch = cpr <= kWave ? 1 : 2;
  int ks = (cpr + nch * kWave - 1) / (nch * kWave);
  if (a.nslots * ks > 16) return VIB3_ERR_UNSUPPORTED;
  a.KS = ks;
  if (a.RB <= 0) a.RB = 16;
  dim3 grid((unsigned)((a.M + a.RB - 1) / a.RB));
  dim3 block((unsigned)(a.nslots * ks * kWave));
  if (nch == 1) hipLaunchKernelGGL((k_down_combine<1>), grid, block, 0, s, a);
  else hipLaunchKernelGGL((k_down_combine<2>), grid, block, 0, s, a);
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
