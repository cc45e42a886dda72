// mxfp4_moe.hip — batched MoE decode over MXFP4 experts as a grouped GEMM on MFMA.
//
// T tokens each pick top_k experts (ids and weights given on the device). Tokens are grouped
// per expert, then every touched expert streams its weights once for all of its tokens:
//   h[t]   = f16( silu(gate_e . x_t) * (up_e . x_t) )     fused gate/up + SwiGLU
//   d[t,j] = f16( down_e . h[t] )
//   out[t] = bf16( sum_j w[t,j] * d[t,j] )                 in pick order, o = o + w*d
// which is the reference's per-token composition (engine.rs:5801-6306 execute_expert, the
// f16 rounding points of kernels.rs:3042 / :2825, weighted_accumulate_f32 kernels.rs:2000)
// applied to MXFP4 weights: E2M1 codes (kernels.cu:438-441, low nibble = even k) times an
// E8M0 scale 2^(e-127) per 32 along k (kernels.cu:2770-2777).
//
// MXFP4 page: [rows x K/2] code bytes, then [rows x K/32] E8M0 bytes.
//
// The contraction runs on the CDNA4 matrix cores: weights are decoded in registers with
// v_cvt_scalef32_pk_{bf16,f16}_fp4 (exact: every E2M1 x 2^e value of the scale range is a
// bf16 / f16 number) and fed to v_mfma_f32_16x16x32_{bf16,f16} against the tokens' bf16
// activations (gate/up) or f16 intermediates (down). Products are exact and accumulate in f32,
// so results differ from the sequential CPU sum only by the order of f32 additions.
#include <hip/hip_ext.h>

#include <mutex>

#include "common.h"
#include "kernels.h"

namespace vib3 {

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

constexpr int kMxTokBlk = 16;            // tokens per MFMA column block (one wave)
constexpr int kMxMaxBlk = 1;             // column blocks per wave
constexpr int kMxChunk = 64;             // tokens of one expert sharing a weight read (4 waves)
constexpr int kMxStep = 256;             // k per step: 2 halves x 4 lane groups x 32
constexpr int kMxTiles = 4;              // 16-row A tiles per wave
constexpr int kMxMaxPicks = 4096;        // tokens * top_k per launch (grouping is one workgroup)
constexpr int kMxColdMax = 2;            // experts with at most this many tokens take the row path

struct MxArgs {
  const uint16_t* x;          // [T][hidden] bf16
  const uint64_t* table;      // [E][3] page addresses: up, gate, down
  const int* d_expert;        // [nd] expert of distinct index d
  const int* d_off;           // [nd] first entry of d
  const int* d_cnt;           // [nd] entries of d
  const int* nd;              // number of distinct experts
  const int* it_d;            // [items] distinct index of each work item
  const int* it_p0;           // [items] first entry of the item's token chunk within its expert
  const int* it_np;           // [items] token blocks of the chunk (1..4) | part << 8
  const int* nitems;
  const int* ent_tok;         // [T*top_k] token of each entry (grouped by expert)
  const int* ent_slot;        // [T*top_k] t*top_k + j of each entry
  const int* c_dix;           // [ncold] distinct index of each cold expert (row path): the
  const int* ncold;           // ncold1 one-token experts first, then the two-token ones
  const int* ncold1;
  uint16_t* h;                // [T*top_k][inter] f16, by entry
  uint16_t* d;                // [T*top_k][hidden] f16, by slot
  int hidden, inter;
};

__device__ __forceinline__ uint4 ld16(const void* p) {
  const u32x4 v = *(const __attribute__((address_space(1))) u32x4*)p;
  return make_uint4(v.x, v.y, v.z, v.w);
}

typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));

__device__ __forceinline__ uint2 ld8(const void* p) {
  const u32x2_t v = *(const __attribute__((address_space(1))) u32x2_t*)p;
  return make_uint2(v.x, v.y);
}

__device__ __forceinline__ uint8_t ld_u8(const uint8_t* p) {
  return *(const __attribute__((address_space(1))) uint8_t*)p;
}

__device__ __forceinline__ float e8m0_scale(uint8_t e) {
  return __uint_as_float((uint32_t)e << 23);
}

// Eight E2M1 codes (one 32-bit word, low nibble first) times `scale` as bf16 / f16 operands.
template <bool BF16>
__device__ __forceinline__ void decode8(uint32_t w, float scale, bf16x8_t& ob, f16x8_t& oh) {
  if (BF16) {
    const bf16x2_t a = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, scale, 0);
    const bf16x2_t b = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, scale, 1);
    const bf16x2_t c = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, scale, 2);
    const bf16x2_t e = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, scale, 3);
    ob = bf16x8_t{a[0], a[1], b[0], b[1], c[0], c[1], e[0], e[1]};
  } else {
    const f16x2_t a = __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(w, scale, 0);
    const f16x2_t b = __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(w, scale, 1);
    const f16x2_t c = __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(w, scale, 2);
    const f16x2_t e = __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(w, scale, 3);
    oh = f16x8_t{a[0], a[1], b[0], b[1], c[0], c[1], e[0], e[1]};
  }
}

// One wave: kMxTiles tiles of 16 weight rows x all the expert's tokens (in passes of 16).
// GATEUP: tiles 0,1 = up rows r0..r0+31, tiles 2,3 = gate rows r0..r0+31 (bf16 MFMA on x);
// otherwise tiles 0..3 = down rows r0..r0+63 (f16 MFMA on h).
//
// Operand layout of v_mfma_f32_16x16x32: lane l supplies A row (l & 15), k block (l >> 4)
// of 8 values, and B column (l & 15), the same k block. Each lane loads the 16 bytes = 32
// codes of its row at k = step*128 + (l >> 4)*32, and MFMA s (0..3) takes the s-th word: the
// four k blocks of one MFMA are then k = step*128 + g*32 + s*8 (g = lane group), a fixed
// permutation of the step's k range that A and B share. The scale of the whole 32-code chunk
// is one E8M0 byte. Result D: lane l holds rows (l >> 4)*4 + i, column l & 15.

template <int NB>
struct MxStep {
  uint4 w[kMxTiles][2];
  uint8_t sc[kMxTiles][2];
  uint4 xb[NB][2][4];
};

// One pass over k for NB column blocks; loads run one step ahead of the matrix-core work.
// A step is 256 k: the lane's 16 bytes at k = ks + g*32 (half 0) and ks + 128 + g*32 (half 1),
// so the four lanes of a row fetch both 64-byte halves of its 128-byte line together.
template <bool GATEUP, int NB>
__device__ __forceinline__ void mx_pass(const uint8_t* const (&tcode)[kMxTiles],
                                        const uint8_t* const (&tscale)[kMxTiles],
                                        const uint16_t* const (&brow)[kMxMaxBlk], int ks0,
                                        int kstride, int nsteps,
                                        f32x4_t (&acc)[kMxTiles][kMxMaxBlk]) {
  auto load = [&](MxStep<NB>& st, int ks) {
#pragma unroll
    for (int t = 0; t < kMxTiles; t++)
#pragma unroll
      for (int h = 0; h < 2; h++) {
        st.w[t][h] = ld16(tcode[t] + ks / 2 + h * 64);
        st.sc[t][h] = ld_u8(tscale[t] + ks / 32 + h * 4);
      }
#pragma unroll
    for (int b = 0; b < NB; b++)
#pragma unroll
      for (int h = 0; h < 2; h++)
#pragma unroll
        for (int s = 0; s < 4; s++) st.xb[b][h][s] = ld16(brow[b] + ks + h * 128 + s * 8);
    __builtin_amdgcn_sched_barrier(0);
  };
  auto compute = [&](const MxStep<NB>& st) {
#pragma unroll
    for (int t = 0; t < kMxTiles; t++) {
#pragma unroll
      for (int h = 0; h < 2; h++) {
        const float scale = e8m0_scale(st.sc[t][h]);
        const uint32_t words[4] = {st.w[t][h].x, st.w[t][h].y, st.w[t][h].z, st.w[t][h].w};
#pragma unroll
        for (int s = 0; s < 4; s++) {
          bf16x8_t ab;
          f16x8_t ah;
          decode8<GATEUP>(words[s], scale, ab, ah);
#pragma unroll
          for (int b = 0; b < NB; b++) {
            if (GATEUP) {
              acc[t][b] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                  ab, __builtin_bit_cast(bf16x8_t, st.xb[b][h][s]), acc[t][b], 0, 0, 0);
            } else {
              acc[t][b] = __builtin_amdgcn_mfma_f32_16x16x32_f16(
                  ah, __builtin_bit_cast(f16x8_t, st.xb[b][h][s]), acc[t][b], 0, 0, 0);
            }
          }
        }
      }
    }
  };
  if (nsteps <= 0) return;
  MxStep<NB> A, B;
  const int last = nsteps - 1;
  load(A, ks0);
  for (int i = 0;; i += 2) {
    load(B, ks0 + min(i + 1, last) * kstride);  // past the end: re-reads the last step
    compute(A);
    if (i + 1 > last) break;
    load(A, ks0 + min(i + 2, last) * kstride);
    compute(B);
    if (i + 2 > last) break;
  }
}

// Work item = (distinct expert, 16-token block of its entries); blockIdx.x = row block.
// A wave owns 4 tiles of 16 rows (gate/up: 32 up rows and the same 32 gate rows; down: 64
// rows) for one token block. With KS = 4 (gate/up, long k) the four waves of a workgroup share
// their tiles and split k: wave w takes the 256-wide steps w, w + 4, ... so at any time the
// workgroup reads four adjacent 128-byte pieces of each of its rows (512 contiguous bytes)
// rather than one piece of each of 128 rows, and the four partial tiles are summed through
// LDS in wave order. With KS = 1 (down, k = 2048 is only 8 steps) the waves take 4 adjacent
// row blocks and each runs its whole k range. The token blocks of one 64-token chunk are
// adjacent items, gridDim.x (for gate/up a multiple of 8) workgroups apart: the same XCD and L2, close in
// time, so HBM serves their shared weight lines once.
template <bool GATEUP, int KS>
__global__ __launch_bounds__(256) void k_mx_gemm(MxArgs a) {
  __shared__ f32x4_t red[KS > 1 ? KS : 1][kMxTiles][kWave];
  const int item = (int)blockIdx.y;
  if (item >= *a.nitems) return;
  const int lane = lane_id();
  const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
  const int rr = lane & 15, g = lane >> 4;
  const int dix = a.it_d[item];
  const int e = a.d_expert[dix], o_e = a.d_off[dix], t_e = a.d_cnt[dix];
  const int part = a.it_np[item] >> 8;
  const int p0 = a.it_p0[item] + part * kMxTokBlk;  // the block's first token (entry index)
  const int K = GATEUP ? a.hidden : a.inter;   // reduction
  const int M = GATEUP ? a.inter : a.hidden;   // rows of each matrix
  const int rpw = GATEUP ? 32 : 64;                 // rows of each matrix per wave
  const int kw = wave % KS;                          // this wave's share of the k steps
  const int r0 = (int)blockIdx.x * rpw * (4 / KS) + (wave / KS) * rpw;
  if (r0 >= M || p0 >= t_e) return;                  // (a guard; uniform when KS > 1)
  const size_t pkb = (size_t)K / 2, nsb = (size_t)K / 32;
  const uint8_t* m0 = (const uint8_t*)a.table[(size_t)e * 3 + (GATEUP ? 0 : 2)];
  const uint8_t* m1 = GATEUP ? (const uint8_t*)a.table[(size_t)e * 3 + 1] : m0;

  // tile t: matrix base and row
  const uint8_t* tcode[kMxTiles];
  const uint8_t* tscale[kMxTiles];
#pragma unroll
  for (int t = 0; t < kMxTiles; t++) {
    const uint8_t* base = GATEUP ? (t < 2 ? m0 : m1) : m0;
    const int row = GATEUP ? r0 + (t & 1) * 16 + rr : r0 + t * 16 + rr;
    tcode[t] = base + (size_t)row * pkb + (size_t)g * 16;
    tscale[t] = base + (size_t)M * pkb + (size_t)row * nsb + g;
  }

  {
    const int nblk = 1;
    // B rows of this lane's column in each block. A column past the expert's tokens reads the
    // block's first token (the same lines as its lane, so no extra traffic): MFMA columns are
    // independent and those columns are never stored.
    const uint16_t* brow[kMxMaxBlk];
#pragma unroll
    for (int b = 0; b < kMxMaxBlk; b++) {
      const int tok0 = p0 + b * kMxTokBlk;
      const int tok = tok0 + rr < t_e ? tok0 + rr : tok0;
      const uint16_t* r =
          GATEUP ? a.x + (size_t)a.ent_tok[o_e + tok] * K : a.h + (size_t)(o_e + tok) * K;
      brow[b] = r + g * 32;
    }
    f32x4_t acc[kMxTiles][kMxMaxBlk];
#pragma unroll
    for (int t = 0; t < kMxTiles; t++)
#pragma unroll
      for (int b = 0; b < kMxMaxBlk; b++) acc[t][b] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    const int nsteps = K / kMxStep;
    mx_pass<GATEUP, kMxMaxBlk>(tcode, tscale, brow, kw * kMxStep, KS * kMxStep,
                               (nsteps - kw + KS - 1) / KS, acc);
    // tiles this wave finishes: all of them (KS = 1), or with KS = 4 tile kw (gate/up: waves
    // 0 and 1 finish row halves 0 and 1 from their up and gate tiles)
    auto mine = [&](int t) { return KS == 1 || (GATEUP ? (t & 1) == kw : t == kw); };
    if (KS > 1) {
      // sum the waves' partial tiles in wave order
#pragma unroll
      for (int t = 0; t < kMxTiles; t++) red[kw][t][lane] = acc[t][0];
      __syncthreads();
      if (GATEUP && kw >= 2) return;
#pragma unroll
      for (int t = 0; t < kMxTiles; t++) {
        if (!mine(t)) continue;
        f32x4_t v = red[0][t][lane];
#pragma unroll
        for (int u = 1; u < KS; u++) {
          const f32x4_t w = red[u][t][lane];
          v = f32x4_t{v[0] + w[0], v[1] + w[1], v[2] + w[2], v[3] + w[3]};
        }
        acc[t][0] = v;
      }
    }

    // epilogue: lane holds rows (g*4 + i) of each tile for token column rr of each block
#pragma unroll
    for (int b = 0; b < kMxMaxBlk; b++) {
      const int tok = p0 + b * kMxTokBlk + rr;
      if (b >= nblk || tok >= t_e) continue;
      if (GATEUP) {
#pragma unroll
        for (int half = 0; half < 2; half++) {
          if (!mine(half)) continue;
          uint16_t hv[4];
#pragma unroll
          for (int i = 0; i < 4; i++) {
            const float up = acc[half][b][i], gate = acc[2 + half][b][i];
            hv[i] = f32_to_f16_bits((gate / (1.0f + expf(-gate))) * up);  // kernels.rs:3041
          }
          const int row = r0 + half * 16 + g * 4;
          uint2 v = make_uint2((uint32_t)hv[0] | ((uint32_t)hv[1] << 16),
                               (uint32_t)hv[2] | ((uint32_t)hv[3] << 16));
          *(uint2*)(a.h + (size_t)(o_e + tok) * M + row) = v;
        }
      } else {
        const int slot = a.ent_slot[o_e + tok];
#pragma unroll
        for (int t = 0; t < kMxTiles; t++) {
          if (!mine(t)) continue;
          uint16_t dv[4];
#pragma unroll
          for (int i = 0; i < 4; i++) dv[i] = f32_to_f16_bits(acc[t][b][i]);
          const int row = r0 + t * 16 + g * 4;
          uint2 v = make_uint2((uint32_t)dv[0] | ((uint32_t)dv[1] << 16),
                               (uint32_t)dv[2] | ((uint32_t)dv[3] << 16));
          *(uint2*)(a.d + (size_t)slot * M + row) = v;
        }
      }
    }
  }
}

// ----------------------------------------------------------------------- matrix-core path, v2
//
// The work items above with the tokens' activations staged in LDS, so a wave can read long
// pieces of few rows: a workgroup of kMx2W = 8 waves owns 128 weight rows (gate/up: 64 up + the
// same 64 gate rows; down: 128 rows), one 16-row tile per wave, and walks k in steps of
// kMx2K = 512. Per step each wave loads 256 contiguous bytes of each of its 16 rows (lane (r, g)
// takes the 16-byte pieces g, g + 4, ... of row r), the workgroup stages the 16 tokens' 512
// activations in LDS once, and the wave runs 16 MFMAs against them. Waves per CU decided the
// rate: per c4 batch, 4-wave workgroups with steps of 1024 (66 KB LDS, 8 waves per CU) took
// 803 us, with steps of 512 (33 KB, 16 waves) 726 us, 8-wave workgroups with steps of 512
// (24 waves per CU) 704 us, and with steps of 256 722 us.
// Loads of step s + 1 (weights into registers, activations
// into the other LDS buffer) are issued before step s's matrix-core work.
#ifndef VIB3_MX2_K
#define VIB3_MX2_K 512  // k per step (build-time tuning knob: 256, 512 or 1024)
#endif
constexpr int kMx2K = VIB3_MX2_K;             // k per step
#ifndef VIB3_MX2_WAVES
#define VIB3_MX2_WAVES 8  // waves per workgroup sharing one activation stage (4 or 8)
#endif
constexpr int kMx2W = VIB3_MX2_WAVES;
constexpr int kMx2H = kMx2W / 2;              // gate/up: waves per matrix
#ifndef VIB3_MX2_KD
#define VIB3_MX2_KD 512  // k per step of the down phase (k = inter; 256 or 512)
#endif
constexpr int kMx2KD = VIB3_MX2_KD;

template <int P>  // P = 16-byte pieces per lane per step
struct Mx2W {
  uint4 w[P];       // 16 bytes of pieces g + 4j, j < P, of this lane's row
  uint32_t sc[P];   // the row's E8M0 scales of the step: byte g of word j = piece g + 4j
};

template <bool GATEUP, int KS>
__global__ __launch_bounds__(64 * kMx2W) void k_mx_gemm2(MxArgs a) {
  constexpr int kP = KS / 128;        // 16-byte pieces per lane per step
  constexpr int kPitch = KS + 8;      // LDS row pitch (halves), against bank conflicts
  static_assert(KS % (32 * kMx2W) == 0 && KS >= 256, "step width");
  __shared__ uint16_t xs[2][kMxTokBlk][kPitch];
  const int item = (int)blockIdx.y;
  if (item >= *a.nitems) return;
  const int tid = (int)threadIdx.x, lane = lane_id();
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int rr = lane & 15, g = lane >> 4;
  const int dix = a.it_d[item];
  const int e = a.d_expert[dix], o_e = a.d_off[dix], t_e = a.d_cnt[dix];
  const int p0 = a.it_p0[item] + (a.it_np[item] >> 8) * kMxTokBlk;

  const int K = GATEUP ? a.hidden : a.inter;
  const int M = GATEUP ? a.inter : a.hidden;
  const int r0 = (int)blockIdx.x * (GATEUP ? 16 * kMx2H : 16 * kMx2W);
  if (p0 >= t_e) return;  // (a guard; uniform)
  const size_t pkb = (size_t)K / 2, nsb = (size_t)K / 32;
  // this wave's tile: gate/up waves 0, 1 = up rows r0 + 16w, waves 2, 3 = gate rows r0 + 16(w-2)
  const int seg = GATEUP ? (wave < kMx2H ? 0 : 1) : 2;
  const int row = GATEUP ? r0 + (wave % kMx2H) * 16 + rr : r0 + wave * 16 + rr;
  const uint8_t* base = (const uint8_t*)a.table[(size_t)e * 3 + seg];
  const uint8_t* code = base + (size_t)row * pkb + (size_t)g * 16;
  const uint8_t* scl = base + (size_t)M * pkb + (size_t)row * nsb;
  // activation staging: each of a token's kParts threads copies kXP x 16 bytes of its row
  constexpr int kParts = 4 * kMx2W;            // staging threads per token
  constexpr int kXP = KS / (32 * kMx2W);    // 16-byte pieces per staging thread
  const int st_tok = tid / kParts, st_part = tid % kParts;
  const int tk = p0 + st_tok;
  const bool st_ok = tk < t_e;
  const uint16_t* xrow =
      GATEUP ? a.x + (size_t)a.ent_tok[o_e + (st_ok ? tk : p0)] * K
             : a.h + (size_t)(o_e + (st_ok ? tk : p0)) * K;
  xrow += st_part * (KS / kParts);

  auto load_w = [&](Mx2W<kP>& w, int k0) {
#pragma unroll
    for (int j = 0; j < kP; j++) w.w[j] = ld16(code + k0 / 2 + j * 64);
    if constexpr (kP >= 4) {
#pragma unroll
      for (int j = 0; j < kP / 4; j++) {
        const uint4 v = ld16(scl + k0 / 32 + 16 * j);
        w.sc[4 * j] = v.x, w.sc[4 * j + 1] = v.y, w.sc[4 * j + 2] = v.z, w.sc[4 * j + 3] = v.w;
      }
    } else {
      const uint2 v = ld8(scl + k0 / 32);
      w.sc[0] = v.x, w.sc[1] = v.y;
    }
  };
  auto load_x = [&](uint4 (&v)[kXP], int k0) {
#pragma unroll
    for (int j = 0; j < kXP; j++) v[j] = ld16(xrow + k0 + j * 8);
  };
  auto store_x = [&](const uint4 (&v)[kXP], int b) {
    uint4* d = (uint4*)&xs[b][st_tok][st_part * (KS / kParts)];
#pragma unroll
    for (int j = 0; j < kXP; j++) d[j] = v[j];
  };
  f32x4_t acc = f32x4_t{0.f, 0.f, 0.f, 0.f};
  auto compute = [&](const Mx2W<kP>& w, int b) {
    const uint32_t* scw = w.sc;
#pragma unroll
    for (int j = 0; j < kP; j++) {
      // piece g + 4j covers k = 128 j + 32 g .. + 31 of the step: E8M0 byte 4j + g
      const float scale = e8m0_scale((uint8_t)(scw[j] >> (8 * g)));
      const uint32_t words[4] = {w.w[j].x, w.w[j].y, w.w[j].z, w.w[j].w};
#pragma unroll
      for (int q = 0; q < 4; q++) {
        bf16x8_t ab;
        f16x8_t ah;
        decode8<GATEUP>(words[q], scale, ab, ah);
        const uint4 xb = *(const uint4*)&xs[b][rr][j * 128 + g * 32 + q * 8];
        if (GATEUP)
          acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ab, __builtin_bit_cast(bf16x8_t, xb), acc,
                                                        0, 0, 0);
        else
          acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah, __builtin_bit_cast(f16x8_t, xb), acc,
                                                       0, 0, 0);
      }
    }
  };

  const int nsteps = K / KS;
  Mx2W<kP> W0, W1;
  uint4 xv[kXP];
  load_w(W0, 0);
  load_x(xv, 0);
  store_x(xv, 0);
  __syncthreads();
  for (int s = 0;; s += 2) {
    // step s from W0 / buffer 0, while step s + 1 loads into W1 / buffer 1
    const bool more1 = s + 1 < nsteps;
    if (more1) {  // activations first: waiting for them must not wait for these weights
      load_x(xv, (s + 1) * KS);
      load_w(W1, (s + 1) * KS);
    }
    compute(W0, 0);
    if (!more1) break;
    store_x(xv, 1);
    __syncthreads();
    const bool more2 = s + 2 < nsteps;
    if (more2) {
      load_x(xv, (s + 2) * KS);
      load_w(W0, (s + 2) * KS);
    }
    compute(W1, 1);
    if (!more2) break;
    store_x(xv, 0);
    __syncthreads();
  }

  // epilogue: lane holds rows g*4 + i of the tile for token column rr
  const int tok = p0 + rr;
  if (GATEUP) {
    // the gate tiles (waves 2, 3) meet the up tiles (waves 0, 1) through LDS
    __syncthreads();
    f32x4_t* ex = (f32x4_t*)&xs[0][0][0];
    if (wave >= kMx2H) ex[(wave - kMx2H) * kWave + lane] = acc;
    __syncthreads();
    if (wave >= kMx2H || tok >= t_e) return;
    const f32x4_t gt = ex[wave * kWave + lane];
    uint16_t hv[4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const float up = acc[i], gate = gt[i];
      hv[i] = f32_to_f16_bits((gate / (1.0f + expf(-gate))) * up);  // kernels.rs:3041
    }
    const int orow = r0 + wave * 16 + g * 4;
    *(uint2*)(a.h + (size_t)(o_e + tok) * M + orow) =
        make_uint2((uint32_t)hv[0] | ((uint32_t)hv[1] << 16), (uint32_t)hv[2] | ((uint32_t)hv[3] << 16));
  } else {
    if (tok >= t_e) return;
    const int slot = a.ent_slot[o_e + tok];
    uint16_t dv[4];
#pragma unroll
    for (int i = 0; i < 4; i++) dv[i] = f32_to_f16_bits(acc[i]);
    const int orow = r0 + wave * 16 + g * 4;
    *(uint2*)(a.d + (size_t)slot * M + orow) =
        make_uint2((uint32_t)dv[0] | ((uint32_t)dv[1] << 16), (uint32_t)dv[2] | ((uint32_t)dv[3] << 16));
  }
}

// ----------------------------------------------------------------------------- row path
//
// Experts picked by at most kMxColdMax tokens (three quarters of the touched experts of a
// Zipf-skewed batch) gain nothing from the matrix cores, whose B operand would be 16 token
// columns of which one or two are real; their cost is streaming the weights. They run as
// multi-token GEMVs: a wave owns a contiguous range of (cold expert, row item) pairs, so it
// streams whole rows front to back (3.5 KB gate/up rows, 1 KB down rows) instead of 128-byte
// pieces of 64 rows, keeps the expert's one or two activation vectors in registers for the
// whole segment, and reduces across lanes once per row.
//
// Lane l holds chunks l, l + 64, ... (16 bytes = 32 codes each, one E8M0 scale per chunk);
// a chunk past the row end reads the row's last chunk and meets zero activations. Codes are
// decoded with v_cvt_scalef32_pk_{bf16,f16}_fp4 (exact) and multiplied into f32 with
// v_dot2_f32_{bf16,f16}. An item is one gate/up row pair (SwiGLU in the epilogue) or four down
// rows; the next item's loads are issued before the current one is reduced.

template <bool GATEUP, int NCH, int NT>
__device__ __forceinline__ void mx_rows_segment(const MxArgs& a, int e, int o_e, int q0, int q1) {
  constexpr int R = GATEUP ? 2 : 4;                // row loads per item
  const int lane = lane_id();
  const int K = GATEUP ? a.hidden : a.inter;
  const int M = GATEUP ? a.inter : a.hidden;
  const int cpr = K / 32;                          // chunks per row
  const size_t pkb = (size_t)K / 2;
  const uint8_t* m0 = (const uint8_t*)ld_table(a.table + (size_t)e * 3 + (GATEUP ? 0 : 2));
  const uint8_t* m1 = GATEUP ? (const uint8_t*)ld_table(a.table + (size_t)e * 3 + 1) : m0;
  const uint8_t* s0 = m0 + (size_t)M * pkb;
  const uint8_t* s1 = m1 + (size_t)M * pkb;

  int ch[NCH];
  bool ok[NCH];
#pragma unroll
  for (int j = 0; j < NCH; j++) {
    ok[j] = lane + 64 * j < cpr;
    ch[j] = ok[j] ? lane + 64 * j : cpr - 1;
  }
  // activations of the segment's tokens: chunk j of token t as 4 x 16 bytes (bf16 or f16)
  uint4 xv[NT][NCH][4];
#pragma unroll
  for (int t = 0; t < NT; t++) {
    const uint16_t* src =
        GATEUP ? a.x + (size_t)a.ent_tok[o_e + t] * K : a.h + (size_t)(o_e + t) * K;
#pragma unroll
    for (int j = 0; j < NCH; j++)
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const uint4 v = ld16(src + (size_t)ch[j] * 32 + i * 8);
        xv[t][j][i] = ok[j] ? v : make_uint4(0u, 0u, 0u, 0u);
      }
  }

  struct Item {
    uint4 w[R][NCH];
    uint8_t sc[R][NCH];
  };
  auto load = [&](Item& it, int q) {
#pragma unroll
    for (int r = 0; r < R; r++) {
      const int row = GATEUP ? q : 4 * q + r;
      const uint8_t* m = GATEUP && r == 1 ? m1 : m0;
      const uint8_t* sp = GATEUP && r == 1 ? s1 : s0;
#pragma unroll
      for (int j = 0; j < NCH; j++) {
        it.w[r][j] = ld_stream(m + (size_t)row * pkb + (size_t)ch[j] * 16);
        it.sc[r][j] = ld_u8(sp + (size_t)row * cpr + ch[j]);
      }
    }
    __builtin_amdgcn_sched_barrier(0);
  };
  auto finish = [&](const Item& it, int q) {
    float acc[R][NT];
#pragma unroll
    for (int r = 0; r < R; r++)
#pragma unroll
      for (int t = 0; t < NT; t++) acc[r][t] = 0.0f;
#pragma unroll
    for (int r = 0; r < R; r++)
#pragma unroll
      for (int j = 0; j < NCH; j++) {
        const float scale = e8m0_scale(it.sc[r][j]);
        const uint32_t wd[4] = {it.w[r][j].x, it.w[r][j].y, it.w[r][j].z, it.w[r][j].w};
#pragma unroll
        for (int i = 0; i < 4; i++) {
          uint32_t wp[4];
          if (GATEUP) {
            wp[0] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(wd[i], scale, 0));
            wp[1] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(wd[i], scale, 1));
            wp[2] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(wd[i], scale, 2));
            wp[3] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(wd[i], scale, 3));
          } else {
            wp[0] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(wd[i], scale, 0));
            wp[1] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(wd[i], scale, 1));
            wp[2] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(wd[i], scale, 2));
            wp[3] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(wd[i], scale, 3));
          }
#pragma unroll
          for (int t = 0; t < NT; t++) {
            const uint32_t xw[4] = {xv[t][j][i].x, xv[t][j][i].y, xv[t][j][i].z, xv[t][j][i].w};
#pragma unroll
            for (int p = 0; p < 4; p++) {
              if (GATEUP)
                acc[r][t] = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, wp[p]),
                                                            __builtin_bit_cast(bf16x2_t, xw[p]),
                                                            acc[r][t], false);
              else
                acc[r][t] = __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2_t, wp[p]),
                                                   __builtin_bit_cast(f16x2_t, xw[p]), acc[r][t],
                                                   false);
            }
          }
        }
      }
#pragma unroll
    for (int r = 0; r < R; r++)
#pragma unroll
      for (int t = 0; t < NT; t++) acc[r][t] = wave_sum(acc[r][t]);
    if (lane < NT) {
#pragma unroll
      for (int t = 0; t < NT; t++) {
        if (t != lane) continue;
        if (GATEUP) {
          const float up = acc[0][t], gate = acc[1][t];
          a.h[(size_t)(o_e + t) * M + q] =
              f32_to_f16_bits((gate / (1.0f + expf(-gate))) * up);  // kernels.rs:3041
        } else {
          const int slot = a.ent_slot[o_e + t];
          const uint2 v = make_uint2(
              (uint32_t)f32_to_f16_bits(acc[0][t]) | ((uint32_t)f32_to_f16_bits(acc[1][t]) << 16),
              (uint32_t)f32_to_f16_bits(acc[2][t]) | ((uint32_t)f32_to_f16_bits(acc[3][t]) << 16));
          *(uint2*)(a.d + (size_t)slot * M + 4 * q) = v;
        }
      }
    }
  };
  Item A, B;
  const int last = q1 - 1;
  load(A, q0);
  for (int q = q0;; q += 2) {
    load(B, min(q + 1, last));  // past the end: re-reads the last item (no branch)
    finish(A, q);
    if (q + 1 > last) break;
    load(A, min(q + 2, last));
    finish(B, q + 1);
    if (q + 2 > last) break;
  }
}

// One launch per token count: the one-token experts' segments hold half the activation
// registers of the two-token ones, so their kernel keeps more waves per SIMD.
template <bool GATEUP, int NCH, int NT>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(NT == 1 && (GATEUP || NCH <= 2) ? 3 : 1)))
void k_mx_rows(MxArgs a) {
  const int n1 = *a.ncold1;
  const int first = NT == 1 ? 0 : n1;
  const int ncold = NT == 1 ? n1 : *a.ncold - n1;
  const int per = GATEUP ? a.inter : a.hidden / 4;  // items per expert
  const long n = (long)ncold * per;
  const int W = (int)gridDim.x * 4;
  const int w = (int)blockIdx.x * 4 + __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
  const long i1 = n * (w + 1) / W;
  for (long i = n * w / W; i < i1;) {
    const int c = (int)(i / per);
    const int q0 = (int)(i - (long)c * per);
    const int q1 = (int)min((long)per, i1 - (long)c * per);
    const int dix = a.c_dix[first + c];
    const int e = a.d_expert[dix], o_e = a.d_off[dix];
    mx_rows_segment<GATEUP, NCH, NT>(a, e, o_e, q0, q1);
    i = (long)c * per + q1;
  }
}

// Token blocks of a chunk of c tokens (1 <= c <= 64).
__host__ __device__ constexpr int mx_chunk_blocks(int c) { return (c + kMxTokBlk - 1) / kMxTokBlk; }

// Work items of an expert with c entries: one per part of each 64-token chunk.
__host__ __device__ inline int mx_expert_items(int c) {
  int n = 0;
  for (int p0 = 0; p0 < c; p0 += kMxChunk) n += mx_chunk_blocks(c - p0 < kMxChunk ? c - p0 : kMxChunk);
  return n;
}

// Group the T*top_k picks by expert (one workgroup). An expert's entries sit in the order its
// counting atomic handed out places: not fixed, and no result depends on it (a token's products
// are formed in its own MFMA column or GEMV lane whatever its place; the combine reads by pick).
// Work items for the GEMM kernels are (distinct expert, 16-token slice of its entries).
struct MxGroupArgs {
  const uint16_t* ids;  // [T*top_k]
  int n, E;
  int* d_expert;
  int* d_off;
  int* d_cnt;
  int* nd;
  int* it_d;            // [items] distinct index of each work item
  int* it_p0;           // [items] first entry (within the expert) of the item's chunk
  int* it_np;           // [items] token blocks of the chunk | part << 8
  int* nitems;
  int* ent_tok;
  int* ent_slot;
  int* c_dix;           // [ncold] distinct index of each expert of the row path (one-token
  int* ncold;           // experts first)
  int* ncold1;
  int top_k;
};

__global__ __launch_bounds__(1024) void k_mx_group(MxGroupArgs a) {
  __shared__ int cnt[kMaxExperts];
  __shared__ int off[kMaxExperts];
  __shared__ int part[1024], dpart[1024], ipart[1024], cpart[1024];
  static_assert(kMxColdMax == 2, "the row path lists one- and two-token experts");
  __shared__ __attribute__((aligned(16))) uint16_t sid[kMxMaxPicks];
  const int tid = (int)threadIdx.x, nt = (int)blockDim.x;
  for (int e = tid; e < a.E; e += nt) cnt[e] = 0;
  for (int p = tid; p < a.n; p += nt) sid[p] = a.ids[p];
  __syncthreads();
  // picks with an id >= E are left out (the combine skips them too)
  // the count's old value is the pick's place among its expert's entries (picks p = tid + k nt;
  // the launch has nt = 1024 threads)
  int myrank[kMxMaxPicks / 1024];
#pragma unroll
  for (int k = 0; k < kMxMaxPicks / 1024; k++) {
    const int p = tid + k * nt;
    myrank[k] = (p < a.n && sid[p] < a.E) ? atomicAdd(&cnt[sid[p]], 1) : 0;
  }
  __syncthreads();
  // exclusive scans over experts of: entries, touched experts, work items. Thread tid owns a
  // contiguous span of experts.
  const int span = (a.E + nt - 1) / nt;
  const int e0 = min(a.E, tid * span), e1 = min(a.E, e0 + span);
  // experts with 1..kMxColdMax entries go to the row path, the others to matrix-core items
  // row-path experts are listed one-token ones first, then two-token ones (one launch each)
  int s = 0, ds = 0, is = 0, c1 = 0, c2 = 0;
  for (int e = e0; e < e1; e++) {
    s += cnt[e];
    ds += cnt[e] > 0;
    is += cnt[e] > kMxColdMax ? mx_expert_items(cnt[e]) : 0;
    c1 += cnt[e] == 1;
    c2 += cnt[e] == 2;
  }
  // inclusive scans of the five counts over the workgroup: within each wave by lane shuffles,
  // then over the (at most 16) wave totals, with two barriers in all
  constexpr int kQ = 5;
  int sc[kQ] = {s, ds, is, c1, c2};
  const int lane = tid & 63, wv = tid >> 6;
#pragma unroll
  for (int st = 1; st < 64; st <<= 1) {
#pragma unroll
    for (int q = 0; q < kQ; q++) {
      const int v = __shfl_up(sc[q], st, 64);
      if (lane >= st) sc[q] += v;
    }
  }
  __shared__ int wtot[16][kQ];
  __shared__ int tot[kQ];
  if (lane == 63) {
#pragma unroll
    for (int q = 0; q < kQ; q++) wtot[wv][q] = sc[q];
  }
  __syncthreads();
  if (tid < kQ) {  // thread q scans the wave totals of count q
    int acc = 0;
    for (int w = 0; w < nt / 64; w++) {
      const int v = wtot[w][tid];
      wtot[w][tid] = acc;  // exclusive: what the waves before w hold
      acc += v;
    }
    tot[tid] = acc;
  }
  __syncthreads();
#pragma unroll
  for (int q = 0; q < kQ; q++) sc[q] += wtot[wv][q];
  part[tid] = sc[0];
  dpart[tid] = sc[1];
  ipart[tid] = sc[2];
  cpart[tid] = tot[3] + tot[4];
  int run = part[tid] - s, drun = dpart[tid] - ds, irun = ipart[tid] - is;
  int c1run = sc[3] - c1, c2run = tot[3] + sc[4] - c2;
  for (int e = e0; e < e1; e++) {
    off[e] = run;
    if (cnt[e] == 1) a.c_dix[c1run++] = drun;
    if (cnt[e] == 2) a.c_dix[c2run++] = drun;
    if (cnt[e] > 0) {
      a.d_expert[drun] = e;
      a.d_off[drun] = run;
      a.d_cnt[drun] = cnt[e];
      for (int p0 = 0; cnt[e] > kMxColdMax && p0 < cnt[e]; p0 += kMxChunk) {
        const int nb = mx_chunk_blocks(min(kMxChunk, cnt[e] - p0));
        for (int part = 0; part < nb; part++) {
          a.it_d[irun] = drun;
          a.it_p0[irun] = p0;
          a.it_np[irun] = nb | (part << 8);
          irun++;
        }
      }
      drun++;
    }
    run += cnt[e];
  }
  if (tid == nt - 1) {
    *a.nd = dpart[nt - 1];
    *a.nitems = ipart[nt - 1];
    *a.ncold = tot[3] + tot[4];
    *a.ncold1 = tot[3];
  }

  __syncthreads();
  // entry position = expert offset + the place the count handed out
#pragma unroll
  for (int k = 0; k < kMxMaxPicks / 1024; k++) {
    const int p = tid + k * nt;
    if (p >= a.n) break;
    const int e = sid[p];
    if (e >= a.E) continue;
    a.ent_tok[off[e] + myrank[k]] = p / a.top_k;
    a.ent_slot[off[e] + myrank[k]] = p;
  }
}

// out[t][r] = bf16(sum_j w[t,j] * d[t,j][r]) in pick order (weighted_accumulate_f32).
__global__ __launch_bounds__(256) void k_mx_combine(const uint16_t* d, const float* w,
                                                      const uint16_t* ids, int E, uint16_t* out,
                                                      int hidden, int top_k) {
  // thread: 8 consecutive outputs of token t. Each group of up to 8 picks has all its loads
  // (ids, weights, 16-byte rows of d) issued before any is used: one round trip per group
  // instead of one per pick.
  const int t = (int)blockIdx.y;
  const int r0 = (int)(blockIdx.x * blockDim.x + threadIdx.x) * 8;
  if (r0 >= hidden) return;
  const bool vec = hidden % 8 == 0 && ((uintptr_t)out & 15) == 0;  // d: the aligned workspace
  float o[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  for (int j0 = 0; j0 < top_k; j0 += 8) {
    uint16_t id[8];
    float wt[8];
    uint4 dv[8];
#pragma unroll
    for (int q = 0; q < 8; q++) {
      const size_t slot = (size_t)t * top_k + min(j0 + q, top_k - 1);
      id[q] = ids[slot];
      wt[q] = w[slot];
      if (vec) {
        dv[q] = *(const uint4*)(d + slot * hidden + r0);
      } else {
        uint16_t h[8];
#pragma unroll
        for (int i = 0; i < 8; i++) h[i] = r0 + i < hidden ? d[slot * hidden + r0 + i] : 0;
        dv[q] = make_uint4(h[0] | (uint32_t)h[1] << 16, h[2] | (uint32_t)h[3] << 16,
                           h[4] | (uint32_t)h[5] << 16, h[6] | (uint32_t)h[7] << 16);
      }
    }
#pragma unroll
    for (int q = 0; q < 8; q++) {
      if (j0 + q >= top_k || id[q] >= E) continue;  // picks past E are skipped
      const uint32_t v[4] = {dv[q].x, dv[q].y, dv[q].z, dv[q].w};
#pragma unroll
      for (int i = 0; i < 4; i++) {
        o[2 * i] = add_mul_rn(o[2 * i], wt[q], f16_to_f32((uint16_t)(v[i] & 0xffff)));
        o[2 * i + 1] = add_mul_rn(o[2 * i + 1], wt[q], f16_to_f32((uint16_t)(v[i] >> 16)));
      }
    }
  }
  // o = o + w * d in pick order per output, as weighted_accumulate_f32 (kernels.rs:2000)
  uint16_t b[8];
#pragma unroll
  for (int i = 0; i < 8; i++) b[i] = f32_to_bf16_bits(o[i]);
  if (vec) {
    *(uint4*)(out + (size_t)t * hidden + r0) =
        make_uint4(b[0] | (uint32_t)b[1] << 16, b[2] | (uint32_t)b[3] << 16,
                   b[4] | (uint32_t)b[5] << 16, b[6] | (uint32_t)b[7] << 16);
  } else {
    for (int i = 0; i < 8 && r0 + i < hidden; i++) out[(size_t)t * hidden + r0 + i] = b[i];
  }
}

// One row-path kernel at its resident grid, cached per instantiation and device (each
// <GATEUP, NCH, NT> variant has its own register budget and therefore its own occupancy).
template <bool GATEUP, int NCH, int NT>
static void mx_launch_rows_one(const MxArgs& a, hipStream_t st) {
  static int grid[64] = {0};
  int dev = 0;
  (void)hipGetDevice(&dev);
  int& g = grid[dev & 63];
  if (!g) g = resident_blocks(k_mx_rows<GATEUP, NCH, NT>, 256);
  hipLaunchKernelGGL((k_mx_rows<GATEUP, NCH, NT>), dim3((unsigned)g), dim3(256), 0, st, a);
}

// Row-path launches (one-token and two-token experts): K = the reduction length picks the
// chunks per lane (K <= 8192).
template <bool GATEUP>
static void mx_launch_rows(const MxArgs& a, int K, hipStream_t st1, hipStream_t st2) {
  switch ((K / 32 + 63) / 64) {
    case 1: mx_launch_rows_one<GATEUP, 1, 1>(a, st1); mx_launch_rows_one<GATEUP, 1, 2>(a, st2); break;
    case 2: mx_launch_rows_one<GATEUP, 2, 1>(a, st1); mx_launch_rows_one<GATEUP, 2, 2>(a, st2); break;
    case 3: mx_launch_rows_one<GATEUP, 3, 1>(a, st1); mx_launch_rows_one<GATEUP, 3, 2>(a, st2); break;
    default: mx_launch_rows_one<GATEUP, 4, 1>(a, st1); mx_launch_rows_one<GATEUP, 4, 2>(a, st2); break;
  }
}

// The two paths are independent until the combine: the matrix-core launches (hot experts) run
// on the caller's stream and the row-path launches (cold experts) on a second stream of the
// library (one per device, default priority), forked after the grouping and joined before the
// combine with events, so each path fills the other's ramps and tails. Enqueueing is
// serialised by a lock (the side stream and its two events are shared by every call on that
// device); under graph capture the fork and join become graph edges.
struct MxSide {
  hipStream_t st = nullptr, st2 = nullptr;  // one-token and two-token row paths
  hipEvent_t fork = nullptr, join = nullptr, join2 = nullptr;
  bool ok = false;
};
#ifndef VIB3_MX_THREE_STREAMS
#define VIB3_MX_THREE_STREAMS 1  // (build-time switch: the two row paths on streams of their own)
#endif
constexpr bool kMxThreeStreams = VIB3_MX_THREE_STREAMS;
// The fork and join events order work of one device only: device-scope fences suffice, and
// skipping the system-scope ones (cache write-back and invalidation at each event) took ~4.5 us
// off a c4 batch.
constexpr unsigned kMxEventFlags = hipEventDisableTiming | hipEventDisableSystemFence;
static MxSide g_mx_side[64];
static std::mutex g_mx_side_lock;

static MxSide* mx_side() {  // called with the lock held
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return nullptr;
  MxSide& s = g_mx_side[dev];
  if (!s.ok) {
    if (hipStreamCreateWithFlags(&s.st, hipStreamNonBlocking) != hipSuccess ||
        hipStreamCreateWithFlags(&s.st2, hipStreamNonBlocking) != hipSuccess)
      return nullptr;
    if (hipEventCreateWithFlags(&s.fork, kMxEventFlags) != hipSuccess ||
        hipEventCreateWithFlags(&s.join, kMxEventFlags) != hipSuccess ||
        hipEventCreateWithFlags(&s.join2, kMxEventFlags) != hipSuccess)
      return nullptr;
    s.ok = true;
  }
  return &s;
}

struct MxWs {
  size_t d_expert, d_off, d_cnt, nd, it_d, it_p0, it_np, nitems, ent_tok, ent_slot, c_dix, ncold, ncold1,
      h, d, total;
};

// Upper bound of the work items: a chunk of c tokens has ceil(c / 16) blocks, at most
// n / 16 + 1 per chunk, and there are at most min(E, n) + n / 64 chunks (a bound with room).
static int mx_max_items(const vib3_moe_mxfp4_batch* B) {
  const int n = B->tokens * B->top_k;
  return n / kMxTokBlk + 2 * ((B->num_experts < n ? B->num_experts : n) + n / kMxChunk);
}

// Grid rows of the matrix-core launches: the work items k_mx_group can form. Each expert there
// has more than kMxColdMax entries and takes ceil(entries / kMxTokBlk) items, so at most
// (n + (kMxTokBlk - 1) m) / kMxTokBlk for m = min(E, n / (kMxColdMax + 1)) such experts. (A
// workgroup past the last item returns at once, but every one of them is still dispatched.)
static int mx_grid_items(const vib3_moe_mxfp4_batch* B) {
  const int n = B->tokens * B->top_k;
  const int hot = n / (kMxColdMax + 1);
  const int m = B->num_experts < hot ? B->num_experts : hot;
  const int bound = (n + (kMxTokBlk - 1) * m) / kMxTokBlk;
  const int cap = mx_max_items(B);
  return bound < cap ? bound : cap;
}

static MxWs mx_ws(const vib3_moe_mxfp4_batch* B) {
  MxWs w{};
  const size_t n = (size_t)B->tokens * B->top_k;
  size_t o = 0;
  auto take = [&](size_t bytes) {
    const size_t at = o;
    o += (bytes + 255) & ~(size_t)255;
    return at;
  };
  w.d_expert = take(sizeof(int) * B->num_experts);
  w.d_off = take(sizeof(int) * B->num_experts);
  w.d_cnt = take(sizeof(int) * B->num_experts);
  w.nd = take(sizeof(int));
  w.it_d = take(sizeof(int) * (size_t)mx_max_items(B));
  w.it_p0 = take(sizeof(int) * (size_t)mx_max_items(B));
  w.it_np = take(sizeof(int) * (size_t)mx_max_items(B));
  w.nitems = take(sizeof(int));
  w.ent_tok = take(sizeof(int) * n);
  w.ent_slot = take(sizeof(int) * n);
  w.c_dix = take(sizeof(int) * B->num_experts);
  w.ncold = take(sizeof(int));
  w.ncold1 = take(sizeof(int));
  w.h = take(2 * n * B->inter);
  w.d = take(2 * n * B->hidden);
  w.total = o;
  return w;
}

}  // namespace vib3

using namespace vib3;

extern "C" {

size_t vib3_moe_mxfp4_workspace_bytes(const vib3_moe_mxfp4_batch* B) {
  if (!B || B->tokens <= 0 || B->top_k <= 0 || B->num_experts <= 0) return 0;
  return mx_ws(B).total;
}

int vib3_launch_moe_mxfp4_batched(const vib3_moe_mxfp4_batch* B, void* stream) {
  if (!B) return VIB3_ERR_BAD_POINTER;
  if (B->tokens <= 0 || B->top_k <= 0 || B->num_experts <= 0 || B->num_experts > kMaxExperts)
    return VIB3_ERR_BAD_COUNT;
  if ((size_t)B->tokens * B->top_k > kMxMaxPicks) return VIB3_ERR_BAD_COUNT;
  if (B->hidden <= 0 || B->inter <= 0 || B->hidden % 256 || B->inter % 256 ||
      B->hidden > 8192 || B->inter > 8192)
    return VIB3_ERR_UNSUPPORTED;  // 256-wide k steps; 256 rows per down workgroup; row path
                                  // holds at most 4 chunks of a row per lane
  if (!B->x || !B->ids || !B->weights || !B->page_table || !B->out || !B->workspace)
    return VIB3_ERR_BAD_POINTER;
  if (((uintptr_t)B->x & 15) || ((uintptr_t)B->workspace & 255)) return VIB3_ERR_BAD_POINTER;
  const MxWs w = mx_ws(B);
  if (B->workspace_bytes < w.total) return VIB3_ERR_WORKSPACE;
  char* ws = (char*)B->workspace;
  hipStream_t st = (hipStream_t)stream;
  const int n = B->tokens * B->top_k;

  MxGroupArgs ga{};
  ga.ids = B->ids; ga.n = n; ga.E = B->num_experts;
  ga.d_expert = (int*)(ws + w.d_expert); ga.d_off = (int*)(ws + w.d_off);
  ga.d_cnt = (int*)(ws + w.d_cnt); ga.nd = (int*)(ws + w.nd);
  ga.ent_tok = (int*)(ws + w.ent_tok); ga.ent_slot = (int*)(ws + w.ent_slot);
  ga.it_d = (int*)(ws + w.it_d); ga.it_p0 = (int*)(ws + w.it_p0); ga.it_np = (int*)(ws + w.it_np);
  ga.nitems = (int*)(ws + w.nitems);
  ga.c_dix = (int*)(ws + w.c_dix); ga.ncold = (int*)(ws + w.ncold);
  ga.ncold1 = (int*)(ws + w.ncold1);
  ga.top_k = B->top_k;
  hipLaunchKernelGGL(k_mx_group, dim3(1), dim3(1024), 0, st, ga);

  MxArgs a{};
  a.x = (const uint16_t*)B->x; a.table = B->page_table;
  a.d_expert = ga.d_expert; a.d_off = ga.d_off; a.d_cnt = ga.d_cnt; a.nd = ga.nd;
  a.it_d = ga.it_d; a.it_p0 = ga.it_p0; a.it_np = ga.it_np; a.nitems = ga.nitems;
  a.ent_tok = ga.ent_tok; a.ent_slot = ga.ent_slot;
  a.c_dix = ga.c_dix; a.ncold = ga.ncold; a.ncold1 = ga.ncold1;
  a.h = (uint16_t*)(ws + w.h); a.d = (uint16_t*)(ws + w.d);
  a.hidden = B->hidden; a.inter = B->inter;
  const unsigned items = (unsigned)mx_grid_items(B);
  std::unique_lock<std::mutex> lock(g_mx_side_lock, std::defer_lock);
  MxSide* side = nullptr;
#ifndef VIB3_MX_ONE_STREAM
#define VIB3_MX_ONE_STREAM 0  // (profiling builds: 1 = the three chains on the caller's stream)
#endif
  if (!VIB3_MX_ONE_STREAM) {
    lock.lock();
    side = mx_side();
  }
  hipStream_t rs = st, rs2 = st;  // the row paths' streams
  if (side) {
    hipError_t e = hipEventRecord(side->fork, st);
    if (e == hipSuccess) e = hipStreamWaitEvent(side->st, side->fork, 0);
    if (e == hipSuccess && kMxThreeStreams) e = hipStreamWaitEvent(side->st2, side->fork, 0);
    if (e != hipSuccess) return (int)e;
    rs = side->st;
    rs2 = kMxThreeStreams ? side->st2 : side->st;
  }
  mx_launch_rows<true>(a, B->hidden, rs, rs2);
  mx_launch_rows<false>(a, B->inter, rs, rs2);
  // matrix-core path: activations staged in LDS when k is a multiple of the step, otherwise
  // registers-only with k split over the waves (gate/up) or whole (down)
  if (items == 0) {  // (no expert can take the matrix-core path)
  } else if (B->hidden % kMx2K == 0)
    hipLaunchKernelGGL((k_mx_gemm2<true, kMx2K>), dim3((unsigned)(B->inter / (16 * kMx2H)), items),
                       dim3(64 * kMx2W), 0,
                       st, a);
  else
    hipLaunchKernelGGL((k_mx_gemm<true, 4>), dim3((unsigned)(B->inter / 32), items), dim3(256), 0,
                       st, a);
  if (items == 0) {
  } else if (B->inter % kMx2KD == 0)
    hipLaunchKernelGGL((k_mx_gemm2<false, kMx2KD>), dim3((unsigned)(B->hidden / (16 * kMx2W)), items),
                       dim3(64 * kMx2W),
                       0, st, a);
  else
    hipLaunchKernelGGL((k_mx_gemm<false, 1>), dim3((unsigned)(B->hidden / 256), items), dim3(256),
                       0, st, a);
  if (side) {
    hipError_t e = hipEventRecord(side->join, rs);
    if (e == hipSuccess) e = hipStreamWaitEvent(st, side->join, 0);
    if (e == hipSuccess && kMxThreeStreams) e = hipEventRecord(side->join2, rs2);
    if (e == hipSuccess && kMxThreeStreams) e = hipStreamWaitEvent(st, side->join2, 0);
    if (e != hipSuccess) return (int)e;
  }
  hipLaunchKernelGGL(k_mx_combine, dim3((unsigned)((B->hidden + 2047) / 2048), (unsigned)B->tokens),
                     dim3(256), 0, st, (const uint16_t*)a.d, B->weights, B->ids,
                     B->num_experts, (uint16_t*)B->out, B->hidden, B->top_k);
  VIB3_RETURN_LAUNCH();
}

}  // extern "C"
