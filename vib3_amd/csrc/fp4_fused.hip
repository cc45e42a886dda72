// fp4_fused.hip — the reference's sync-free fused MoE over NVFP4 pages (E2M1 weights with
// per-32 block scales, FP4-quantized activations), rebuilt for gfx950:
//   vib3_launch_quantize_activation_fp4[_fast]  (kernels.cu:3193-3266, :5252)
//   vib3_launch_moe_experts_fused[_gpu]          (kernels.cu:5650, :5868; cuda_ffi.rs:809, :831)
//   vib3_moe_prewarm_gpu_bufs                    (kernels.cu:6507; cuda_ffi.rs:1026)
//   vib3_launch_repack_weights_inplace           (kernels.cu:4132-4183; cuda_ffi.rs:662)
//   vib3_launch_repack_row_to_tiled              (kernels.cu:4185-4262; cuda_ffi.rs:718)
//
// Data formats (the contract of the reference's pages and activations):
//   * split-half E2M1: per group of 32 values, 16 bytes; byte j holds value j in its low
//     nibble and value j + 16 in its high nibble (kernels.cu:4125-4131);
//   * tiled weight data: 16-row x 64-column tiles of 512 bytes, tile (rb, t) at
//     (rb * K/64 + t) * 512, row r of the tile at + 32 r, its two groups at +0 / +16
//     (kernels.cu:4185-4197);
//   * weight scales after the data: [rows][K/32] 2-byte values read as E8M0 = (s >> 7) & 0xff,
//     the exponent byte of a bf16 (kernels.cu:5404-5411); activation scales: E8M0 bytes;
//   * E8M0 e is the power of two 2^(e - 127) (kernels.cu:2770-2777).
//
// Arithmetic: a group's dot product of 32 E2M1 x E2M1 products is an exact multiple of 1/4
// (|.| <= 1152), so it is formed exactly in f32 with v_dot2_f32_f16 on decoded pairs, scaled by
// the exact power of two 2^(ew + ea - 254) and accumulated in f64; the row sum is rounded to
// f32 once. The result is therefore independent of the summation order (the reference sums
// with MMA and K-parallel atomics, whose order varies run to run) and equals the oracle's
// exactly. SwiGLU uses a Cody-Waite / Taylor exp of this file (the same operations as the
// oracle, no contraction), so the FP4 intermediate is bit-identical to the oracle's too.
#include <mutex>

#include "common.h"
#include "fp4.h"
#include "kernels.h"

namespace vib3 {
namespace {

// ------------------------------------------------------------------------- arguments

struct Fp4Mat {
  const uint8_t* data;     // tiled split-half codes
  const uint16_t* scales;  // [rows][K/32]
};

struct Fp4Args {
  const uint8_t* act;     // [K_in/2] split-half codes of the activation
  const uint8_t* act_sc;  // [K_in/32] E8M0
  // device-table form (moe_experts_fused_gpu): page = table[(layer * E + id) * 3 + seg]
  const uint64_t* table;
  const uint16_t* ids;
  const float* wts_dev;
  int layer, E;
  // host-pointer form (moe_experts_fused): per slot up, gate, down
  Fp4Mat mat[kFp4MaxActive][3];
  float wts[kFp4MaxActive];
  int n;                  // active experts
  int K_in, M_mid, M_out;
  // per slot (stride mid_stride): [M_mid/2] codes, [M_mid/32] E8M0, and in the stride's last
  // 16 bytes the slot's down record {data, scales} (both 0 for an unusable slot), written by
  // the gate/up kernel so the down kernel reads its page addresses in one round trip
  uint8_t* mid;
  size_t mid_stride;
  float* out;             // [M_out] += sum_e w_e * down_e(h_e)
};

constexpr int kDownRecord = 16;  // bytes of a slot's down record in the intermediate buffer

// Matrix `seg` of slot s, or {null, null} when the slot's id or page is not usable.
__device__ __forceinline__ Fp4Mat slot_mat(const Fp4Args& a, int s, int seg, int rows, int K) {
  if (!a.table) return a.mat[s][seg];
  const int id = (int)a.ids[s];
  if (id >= a.E) return Fp4Mat{nullptr, nullptr};
  const uint64_t page = a.table[((size_t)a.layer * a.E + id) * 3 + seg];
  if (!page) return Fp4Mat{nullptr, nullptr};
  const uint8_t* p = (const uint8_t*)(uintptr_t)page;
  return Fp4Mat{p, (const uint16_t*)(p + (size_t)(K / 2) * rows)};
}

// The three matrices of slot s for a workgroup-uniform s, as slot_mat gives them: the id (the
// aligned word that holds it) and the table row through scalar loads, one round trip each,
// shared by the three.
__device__ __forceinline__ void slot_mats(const Fp4Args& a, int s, Fp4Mat (&m)[3]) {
  if (!a.table) {
#pragma unroll
    for (int g = 0; g < 3; g++) m[g] = a.mat[s][g];
    return;
  }
  const uintptr_t pid = (uintptr_t)(a.ids + s);
  const uint32_t w = *(const __attribute__((address_space(4))) uint32_t*)(pid & ~(uintptr_t)3);
  const int id = (int)((pid & 2) ? (w >> 16) : (w & 0xffffu));
  const uint64_t* row = a.table + ((size_t)a.layer * a.E + (id < a.E ? id : 0)) * 3;
  const uint64_t pg[3] = {ld_table(row), ld_table(row + 1), ld_table(row + 2)};
#pragma unroll
  for (int g = 0; g < 3; g++) {
    const int rows = g < 2 ? a.M_mid : a.M_out, K = g < 2 ? a.K_in : a.M_mid;
    const uint8_t* p = (const uint8_t*)(uintptr_t)pg[g];
    m[g] = id < a.E && pg[g] ? Fp4Mat{p, (const uint16_t*)(p + (size_t)(K / 2) * rows)}
                             : Fp4Mat{nullptr, nullptr};
  }
}

// Decode split-half groups (codes + E8M0 bytes) into LDS pairs and exponents: group g of
// `groups` goes to lds_pairs[g * 4 .. g * 4 + 3] / lds_exp[g]. Staging is split so the caller can
// issue its first weight loads between the loads of the first R groups per thread (issue) and
// their conversion (finish); finish() then stages any remaining groups directly.
template <int R>
struct Stage {
  uint4 w[R];
  uint8_t e[R];
  const uint8_t* codes;
  const uint8_t* sc;
  int groups;

  __device__ __forceinline__ void issue(const uint8_t* c, const uint8_t* s_, int n) {
    codes = c;
    sc = s_;
    groups = n;
#pragma unroll
    for (int r = 0; r < R; r++) {
      const int g = min((int)threadIdx.x + r * (int)blockDim.x, n - 1);
      w[r] = *(const uint4*)(codes + (size_t)g * 16);
      e[r] = sc[g];
    }
    __builtin_amdgcn_sched_barrier(0);  // these loads go out before anything issued later
  }
  __device__ __forceinline__ static void put(uint4* lds_pairs, int* lds_exp, int g, uint4 w,
                                             uint8_t e) {
    f16x2 p[16];
    decode_group(w, p);
#pragma unroll
    for (int q = 0; q < 4; q++)
      lds_pairs[(size_t)g * 4 + q] =
          make_uint4(__builtin_bit_cast(uint32_t, p[4 * q]), __builtin_bit_cast(uint32_t, p[4 * q + 1]),
                     __builtin_bit_cast(uint32_t, p[4 * q + 2]), __builtin_bit_cast(uint32_t, p[4 * q + 3]));
    lds_exp[g] = (int)e;
  }
  __device__ __forceinline__ void finish(uint4* lds_pairs, int* lds_exp) {
#pragma unroll
    for (int r = 0; r < R; r++) {
      const int g = (int)threadIdx.x + r * (int)blockDim.x;
      if (g < groups) put(lds_pairs, lds_exp, g, w[r], e[r]);
    }
    for (int g = (int)threadIdx.x + R * (int)blockDim.x; g < groups; g += (int)blockDim.x)
      put(lds_pairs, lds_exp, g, *(const uint4*)(codes + (size_t)g * 16), sc[g]);
  }
};

// Stream of one 16-row block of a tiled matrix over tile pairs [p0, p1): lane l owns row
// l & 15 and, within each 1 KB pair of tiles, group (l >> 4), whose 16 bytes sit at
// (gg >> 1) * 512 + row * 32 + (gg & 1) * 16, so one load instruction reads the pair's whole
// kilobyte. The block's scales for the range (16 rows x ng = 4 (p1 - p0) groups, row-major in
// memory) are read once, coalesced, two per lane-word, and kept as E8M0 bytes in LDS (se):
// read per pair, they would cost one scattered 16-line load per kilobyte of weights.
// D pairs are in flight; start() issues the first D before the caller stages its activations,
// step() reduces one while issuing the next. The lane's f64 partial sum is exact.
constexpr int kScaleRegs = 8;  // scale words per lane held across the prologue (ng <= 64)

template <int D>
struct PairStream {
  const uint8_t* base;
  const uint16_t* sc0;  // scale of row rb * 16 + r, group 4 p0 + j at sc0[r * G + j]
  uint8_t* se;          // LDS [16][ng] E8M0 bytes
  int G, ng, p0, p1, gg, row;
  uint4 w[D];
  uint32_t sr[kScaleRegs];

  __device__ __forceinline__ void init(const Fp4Mat m, int rb, int nkt, int G_, int q0, int q1,
                                       uint8_t* lds_e) {
    const int lane = lane_id();
    row = lane & 15;
    gg = lane >> 4;
    G = G_;
    p0 = q0;
    p1 = q1;
    ng = 4 * (q1 - q0);
    base = m.data + ((size_t)rb * nkt) * 512 + (gg >> 1) * 512 + row * 32 + (gg & 1) * 16;
    sc0 = m.scales + (size_t)rb * 16 * G + 4 * q0;
    se = lds_e;
  }
  // scale word i of the range: row i / (ng / 2), groups 2 (i % (ng / 2)) and the next
  __device__ __forceinline__ const uint32_t* scale_word(int i) const {
    const int h = max(ng / 2, 1), r = i / h, j = i - r * h;
    return (const uint32_t*)(sc0 + (size_t)r * G + 2 * j);
  }
  __device__ __forceinline__ void issue_scales() {
    const int n = 8 * ng;  // words: 16 rows x ng / 2
#pragma unroll
    for (int k = 0; k < kScaleRegs; k++) {
      const int i = min(lane_id() + 64 * k, max(n - 1, 0));
      sr[k] = *(const __attribute__((address_space(1))) uint32_t*)scale_word(i);
    }
    __builtin_amdgcn_sched_barrier(0);
  }
  __device__ __forceinline__ void put_word(int i, uint32_t v) {
    const int h = max(ng / 2, 1), r = i / h, j = i - r * h;
    se[r * ng + 2 * j] = (uint8_t)(v >> 7);
    se[r * ng + 2 * j + 1] = (uint8_t)(v >> 23);
  }
  __device__ __forceinline__ void finish_scales() {
    const int n = 8 * ng;
#pragma unroll
    for (int k = 0; k < kScaleRegs; k++)
      if (lane_id() + 64 * k < n) put_word(lane_id() + 64 * k, sr[k]);
    for (int i = lane_id() + 64 * kScaleRegs; i < n; i += 64) put_word(i, *scale_word(i));
  }
  // pair p into buffer d (a pair past the end re-reads the last valid one: no branch around
  // the load, so every step issues one load and the waits below stay exact)
  __device__ __forceinline__ void issue(int d, int p) {
    const int q = max(p < p1 ? p : p1 - 1, 0);
    w[d] = ld_stream(base + (size_t)q * 1024);
    __builtin_amdgcn_sched_barrier(0);
  }
  __device__ __forceinline__ void start() {
#pragma unroll
    for (int d = 0; d < D; d++) issue(d, p0 + d);
  }
  // reduce pair p (in buffer d) into acc (p past the end: nothing) and refill the buffer with
  // pair p + D
  __device__ __forceinline__ void step(int d, int p, const uint4* act_pairs, const int* act_exp,
                                       double& acc) {
    const int pc = min(p, p1 - 1);
    const int g = 4 * pc + gg;
    const float sdot = group_dot(w[d], act_pairs + (size_t)g * 4);
    const int ew = se[row * ng + 4 * (pc - p0) + gg];
    const double t = fma((double)sdot, pow2d(ew + act_exp[g] - 254), acc);
    acc = p < p1 ? t : acc;
    issue(d, p + D);
  }
};

// NS streams over the same pairs (one, or up and gate of a block), interleaved: every step of
// every stream issues one load, so before a step the loads still allowed in flight are those
// of the NS * D - 1 steps issued after the buffer it reads.
template <int D, int NS>
__device__ __forceinline__ void run_streams(PairStream<D> (&st)[NS], const uint4* act_pairs,
                                            const int* act_exp, double (&acc)[NS]) {
#pragma unroll
  for (int i = 0; i < NS; i++) acc[i] = 0.0;
  const int p0 = st[0].p0, p1 = st[0].p1;
  for (int b = p0; b < p1; b += D) {
#pragma unroll
    for (int d = 0; d < D; d++) {
#pragma unroll
      for (int i = 0; i < NS; i++) {
        VIB3_WAIT_VM(NS * D - 1);
        st[i].step(d, b + d, act_pairs, act_exp, acc[i]);
      }
    }
  }
}

// ------------------------------------------------------------------------- kernels

// Down projection + weighted combine, one workgroup per CU: wave w owns the four output rows
// 4 rg .. 4 rg + 3 (rg = the wave's row group) of every slot and walks the slots in order, so
// each row's o = o + w_s * f32(d_s) is formed in registers in slot order (kernels.cu:5958-5990
// accumulates the same terms). A step reads, for the wave's four rows, the 128 contiguous bytes
// they hold in each of 8 J consecutive 512-byte tiles: lane l takes tiles (l >> 3) + 8 j, row
// (l >> 1) & 3 and half l & 1, i.e. J 32-value groups, each reduced exactly (group_dot)
// against the slot's staged intermediate and accumulated in f64 with its two E8M0 scales. The
// slots' intermediates are staged in LDS once per workgroup; page addresses sit in lanes
// (lane s: slot s, from the slot's down record). Needs M_mid % (512 J) == 0.
#ifndef VIB3_FP4_DOWN_NB
#define VIB3_FP4_DOWN_NB 2
#endif

template <int J>
__global__ __launch_bounds__(1024) void k_fp4_down_rows(Fp4Args a) {
  VIB3_TRACE_POINT(0);
  // the kernel arguments the prologue reads, requested together (one round trip)
  asm volatile("" ::"s"(a.n), "s"(a.M_mid), "s"(a.M_out), "s"(a.mid), "s"(a.mid_stride),
               "s"(a.table), "s"(a.wts_dev), "s"((int)blockDim.x));
  extern __shared__ uint4 lds[];
  const int Gm = a.M_mid / 32, nkt = a.M_mid / 64, S8 = nkt / (8 * J), n = a.n;
  uint4* hp = lds;                               // [n][Gm][4]
  int* he = (int*)(lds + (size_t)n * Gm * 4);    // [n][Gm]
  const int lane = lane_id();
  const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
  const int G4 = a.M_out / 4;
  const int rg = (int)blockIdx.x * (int)(blockDim.x >> 6) + wave;
  const int rgc = min(rg, G4 - 1);
  const int rb = rgc >> 2, rs = rgc & 3;
  const int t = lane >> 3, r = (lane >> 1) & 3, hh = lane & 1;
  const int row = rb * 16 + rs * 4 + r;
  // lane s < n: slot s's down record (data, scales; 0 for an unusable slot), first
  uint64_t my_d = 0, my_q = 0;
  if (lane < n) {
    const uint4 rec = *(const uint4*)(a.mid + (size_t)(lane + 1) * a.mid_stride - kDownRecord);
    my_d = ((uint64_t)rec.y << 32) | rec.x;
    my_q = ((uint64_t)rec.w << 32) | rec.z;
  }
  // every slot's intermediate: loads first (thread-strided groups of all slots)
  const int ngr = n * Gm;
  uint4 hw[2];
  uint8_t hx[2];
#pragma unroll
  for (int u = 0; u < 2; u++) {
    const int g = min((int)threadIdx.x + u * (int)blockDim.x, ngr - 1), sl = g / Gm,
              gi = g - sl * Gm;
    const uint8_t* hc = a.mid + (size_t)sl * a.mid_stride;
    hw[u] = *(const uint4*)(hc + (size_t)gi * 16);
    hx[u] = hc[a.M_mid / 2 + gi];
  }
  // lane s < n: slot s's routing weight; ok = 0 for an unusable slot
  float my_w = 0.0f;
  if (lane < n) my_w = a.table ? a.wts_dev[lane] : a.wts[lane];
  const int my_ok = (my_d != 0) & (my_q != 0);
  auto rl64 = [&](uint64_t v, int l) {
    return ((uint64_t)(uint32_t)__builtin_amdgcn_readlane((int)(v >> 32), l) << 32) |
           (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)v, l);
  };
  const int total = n * S8;
  struct Step {
    uint4 w[J];
    uint16_t q[J];
  };
  // step i = (slot i / S8, tiles (i % S8) 8 J ..); past the end or an unusable slot: the same
  // loads from the intermediate buffer (no branch around the loads)
  auto issue = [&](int i, Step& st) {
    const int sl = min(i / S8, n - 1), s8 = i - (i / S8) * S8;
    const bool ok = i < total && __builtin_amdgcn_readlane(my_ok, sl);
    const uint8_t* d = (const uint8_t*)(uintptr_t)rl64(my_d, sl);
    const uint16_t* qs = (const uint16_t*)(uintptr_t)rl64(my_q, sl);
#pragma unroll
    for (int j = 0; j < J; j++) {
      const int kt = s8 * 8 * J + t + 8 * j;
      const uint8_t* pw =
          ok ? d + ((size_t)rb * nkt + kt) * 512 + (rs * 4 + r) * 32 + hh * 16 : a.mid;
      const uint16_t* pq = ok ? qs + (size_t)row * Gm + 2 * kt + hh : (const uint16_t*)a.mid;
      st.w[j] = ld_stream(pw);
      st.q[j] = ld_u16(pq);
    }
    __builtin_amdgcn_sched_barrier(0);
  };
  constexpr int NB = VIB3_FP4_DOWN_NB;  // steps in the ring (NB - 1 in flight while one reduces)
  Step bs[NB];
#pragma unroll
  for (int b = 0; b + 1 < NB; b++) issue(b, bs[b]);
  VIB3_TRACE_POINT(1);  // first steps issued
  // Every lane takes delivery of its intermediate words here, outside the masked region below
  // (a wait inside it would leave the compiler unsure whether they are done, and it would
  // then wait for the weight loads as well).
#pragma unroll
  for (int u = 0; u < 2; u++)
    asm volatile("" ::"v"(hw[u].x), "v"(hw[u].y), "v"(hw[u].z), "v"(hw[u].w), "v"((uint32_t)hx[u]));
  // stage: the first two groups per thread from registers, the rest directly
#pragma unroll
  for (int u = 0; u < 2; u++) {
    const int g = (int)threadIdx.x + u * (int)blockDim.x;
    if (g < ngr) {
      const int sl = g / Gm, gi = g - sl * Gm;
      Stage<1>::put(hp + (size_t)sl * Gm * 4, he + (size_t)sl * Gm, gi, hw[u], hx[u]);
    }
  }
  for (int g = (int)threadIdx.x + 2 * (int)blockDim.x; g < ngr; g += (int)blockDim.x) {
    const int sl = g / Gm, gi = g - sl * Gm;
    const uint8_t* hc = a.mid + (size_t)sl * a.mid_stride;
    Stage<1>::put(hp + (size_t)sl * Gm * 4, he + (size_t)sl * Gm, gi,
                  *(const uint4*)(hc + (size_t)gi * 16), hc[a.M_mid / 2 + gi]);
  }
  __syncthreads();
  VIB3_TRACE_POINT(2);  // intermediates staged
  if (rg >= G4) return;
  float o = a.out[row];
  double acc = 0.0;
  for (int i = 0; i < total; i += NB) {
#pragma unroll
    for (int b = 0; b < NB; b++) {
      const int k = i + b;
      VIB3_WAIT_VM((NB - 2) * 2 * J);  // step k's loads done
      issue(k + NB - 1, bs[(b + NB - 1) % NB]);
      const int sl = min(k / S8, n - 1), s8 = k - (k / S8) * S8;
#pragma unroll
      for (int j = 0; j < J; j++) {
        const int g = 2 * (s8 * 8 * J + t + 8 * j) + hh;
        const float sdot = group_dot(bs[b].w[j], hp + ((size_t)sl * Gm + g) * 4);
        const int ew = (bs[b].q[j] >> 7) & 0xff;
        const double tt = fma((double)sdot, pow2d(ew + he[sl * Gm + g] - 254), acc);
        acc = k < total ? tt : acc;
      }
      if (s8 == S8 - 1 && k < total) {  // the slot's last step: its row sums, in order
        double v = acc;
        v += shfl_xor_d(v, 1);
        v += shfl_xor_d(v, 8);
        v += shfl_xor_d(v, 16);
        v += shfl_xor_d(v, 32);
        const float wsl = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(my_w), sl));
        const float nv = add_mul_rn(o, wsl, (float)v);
        o = __builtin_amdgcn_readlane(my_ok, sl) ? nv : o;
        acc = 0.0;
      }
#ifdef VIB3_TRACE
      if (k == 0) VIB3_TRACE_POINT(3);  // first step reduced
#endif
    }
  }
  VIB3_TRACE_POINT(4);  // loop end
  if (t == 0 && hh == 0) a.out[row] = o;
}

// Activation quantizer (kernels.cu:3193-3240): per group of 32, E8M0 from the absolute maximum,
// values times 1/scale rounded to E2M1, packed split-half. One lane per value: each 32-lane
// half of a wave is one group; lane j < 16 of the group writes byte j = code j | code j+16.
__global__ __launch_bounds__(256) void k_fp4_quant_act(const float* x, uint8_t* codes,
                                                       uint8_t* scales, int K) {
  const int i = (int)(blockIdx.x * blockDim.x + threadIdx.x);
  const int lane = lane_id();
  const float v = i < K ? x[i] : 0.0f;
  float amax = fabsf(v);
#pragma unroll
  for (int m = 1; m < 32; m <<= 1) amax = fmaxf(amax, __shfl_xor(amax, m));
  const uint32_t e = e8m0_of_amax(amax);
  const float inv = amax == 0.0f ? 0.0f : e8m0_inv(e);
  const uint32_t code = e2m1_rne(v * inv);
  const uint32_t hi = (uint32_t)__shfl(code, (lane & ~31) + (lane & 15) + 16);
  const int g = i >> 5, j = i & 31;
  if (j < 16 && g * 32 + j < K) codes[(size_t)g * 16 + j] = (uint8_t)(code | (hi << 4));
  if (j == 0 && g * 32 < K) scales[g] = (uint8_t)e;
}

// Weight quantizer (kernels.cu:6017-6128): f16 [M][K] (K a multiple of 32, so every group lies
// in one row and the groups of the flattened matrix are its rows' groups in order) to
// row-major split-half E2M1 codes and bf16 scales holding the E8M0 exponent (e << 7), the
// format of the block-scaled GEMV kernels. The same rule per group as k_fp4_quant_act.
__global__ __launch_bounds__(256) void k_fp4_weight_quant(const uint16_t* w, uint8_t* codes,
                                                          uint16_t* scales, long long n) {
  const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  const int lane = lane_id();
  const float v = i < n ? f16_to_f32(w[i]) : 0.0f;
  float amax = fabsf(v);
#pragma unroll
  for (int m = 1; m < 32; m <<= 1) amax = fmaxf(amax, __shfl_xor(amax, m));
  const uint32_t e = e8m0_of_amax(amax);
  const float inv = amax == 0.0f ? 0.0f : e8m0_inv(e);
  const uint32_t code = e2m1_rne(v * inv);
  const uint32_t hi = (uint32_t)__shfl(code, (lane & ~31) + (lane & 15) + 16);
  const long long g = i >> 5;
  const int j = (int)(i & 31);
  if (j < 16 && i < n) codes[g * 16 + j] = (uint8_t)(code | (hi << 4));
  if (j == 0 && i < n) scales[g] = (uint16_t)(e << 7);
}

// Fused RMSNorm + FP4 quantizer (kernels.cu:6585-6702). Every workgroup forms the inverse RMS
// in the reference's order: thread t accumulates x[d]^2 (fused multiply-adds) for d = t + 256 i,
// each 32-thread half-wave sums by the butterfly xor 16 .. 1, and the eight half-wave sums
// are added in order from 0; inv = 1 / sqrtf(ss / K + eps), correctly rounded (the reference
// uses CUDA's approximate rsqrtf). Workgroup b then normalises and quantizes elements
// [1024 b, 1024 b + 1024): y = (x * inv) * w, one lane per value as k_fp4_quant_act, and
// optionally writes y as f16.
__global__ __launch_bounds__(256) void k_fp4_rms_quant(const float* x, const uint16_t* w,
                                                       uint8_t* codes, uint8_t* scales,
                                                       uint16_t* f16_out, int K, float eps) {
  __shared__ float ws[8];
  const int tid = (int)threadIdx.x, lane = lane_id();
  float p = 0.0f;
  if (K <= 256 * 32) {
    float v[32];
#pragma unroll
    for (int i = 0; i < 32; i++) v[i] = tid + 256 * i < K ? x[tid + 256 * i] : 0.0f;
#pragma unroll
    for (int i = 0; i < 32; i++) p = tid + 256 * i < K ? __builtin_fmaf(v[i], v[i], p) : p;
  } else {
    for (int d = tid; d < K; d += 256) p = __builtin_fmaf(x[d], x[d], p);
  }
#pragma unroll
  for (int m = 16; m > 0; m >>= 1) p += __shfl_xor(p, m);
  if ((tid & 31) == 0) ws[tid >> 5] = p;
  __syncthreads();
  float total = 0.0f;
#pragma unroll
  for (int i = 0; i < 8; i++) total += ws[i];
  const float inv = 1.0f / __builtin_sqrtf(total / (float)K + eps);
#pragma unroll
  for (int it = 0; it < 4; it++) {
    const int i = (int)blockIdx.x * 1024 + it * 256 + tid;
    float y = 0.0f;
    if (i < K) {
#pragma clang fp contract(off)
      y = x[i] * inv * f16_to_f32(w[i]);
      if (f16_out) f16_out[i] = f32_to_f16_bits(y);
    }
    float amax = fabsf(y);
#pragma unroll
    for (int m = 1; m < 32; m <<= 1) amax = fmaxf(amax, __shfl_xor(amax, m));
    const uint32_t e = e8m0_of_amax(amax);
    const float is = amax == 0.0f ? 0.0f : e8m0_inv(e);
    const uint32_t code = e2m1_rne(y * is);
    const uint32_t hi = (uint32_t)__shfl(code, (lane & ~31) + (lane & 15) + 16);
    const int g = i >> 5, j = i & 31;
    if (j < 16 && i < K) codes[(size_t)g * 16 + j] = (uint8_t)(code | (hi << 4));
    if (j == 0 && i < K) scales[g] = (uint8_t)e;
  }
}

// Gate/up of every active expert + SwiGLU + FP4 quantization of h (kernels.cu:5357-5517 fused):
// workgroup (q, s) = 32 rows [32q, 32q + 32) of slot s; wave w takes row block 2q + (w >> 2)
// and k quarter w & 3 of both matrices; the quarters meet in LDS, and the 32 rows, one E8M0
// group of h, are quantized and written split-half.
#ifdef VIB3_TRACE  // (2-D grid: one probe row per workgroup, y-major)
#define FP4_TRACE(k)                                                                     \
  do {                                                                                   \
    if (threadIdx.x == 0)                                                                \
      vib3_trace_buf[(blockIdx.y * gridDim.x + blockIdx.x) * 16 + (k)] =                 \
          __builtin_amdgcn_s_memrealtime();                                              \
  } while (0)
#else
#define FP4_TRACE(k) \
  do {               \
  } while (0)
#endif

__global__ __launch_bounds__(512) void k_fp4_gateup(Fp4Args a) {
  FP4_TRACE(0);
  extern __shared__ uint4 lds[];
  const int Gin = a.K_in / 32, nkt = a.K_in / 64, P = nkt / 2;
  uint4* act_pairs = lds;                               // [Gin][4]
  int* act_exp = (int*)(lds + (size_t)Gin * 4);         // [Gin]
  __shared__ double part[8][16][2];
  __shared__ float hrow[32];
  const int s = (int)blockIdx.y, q = (int)blockIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
  const int lane = lane_id();
  // the kernel arguments the prologue reads, requested together (one round trip)
  asm volatile("" ::"s"(a.table), "s"(a.ids), "s"(a.E), "s"(a.layer), "s"(a.K_in), "s"(a.M_mid),
               "s"(a.M_out), "s"(a.mid), "s"(a.mid_stride), "s"(a.act), "s"(a.act_sc),
               "s"((int)blockDim.x));
  Fp4Mat mats[3];
  slot_mats(a, s, mats);
  const Fp4Mat up = mats[0], gate = mats[1];
  uint8_t* hcodes = a.mid + (size_t)s * a.mid_stride;
  uint8_t* hsc = hcodes + a.M_mid / 2;
  // workgroup (0, s) also writes slot s's down record (stored at its end: no wait for it here)
  const Fp4Mat dn = mats[2];
  auto put_record = [&]() {
    if (q == 0 && threadIdx.x == 0) {
      const bool ok = dn.data && dn.scales;
      uint64_t* rec = (uint64_t*)(hcodes + a.mid_stride - kDownRecord);
      rec[0] = ok ? (uint64_t)(uintptr_t)dn.data : 0;
      rec[1] = ok ? (uint64_t)(uintptr_t)dn.scales : 0;
    }
  };
  if (!up.data || !gate.data || !up.scales || !gate.scales) {  // unusable slot: h = 0
    if (threadIdx.x < 16) hcodes[(size_t)q * 16 + threadIdx.x] = 0;
    if (threadIdx.x == 0) hsc[q] = 0;
    put_record();
    return;
  }
  const int rb = 2 * q + (wave >> 2), kq = wave & 3;
  const int p0 = kq * P / 4, p1 = (kq + 1) * P / 4;
  const int ngmax = 4 * ((P + 3) / 4);
  uint8_t* se = (uint8_t*)(act_exp + Gin) + (size_t)wave * 2 * 16 * ngmax;
  // staging and scale loads first, then the first weight loads, then the conversions (which
  // wait only for the staging and scale loads)
  Stage<2> stage;
  stage.issue(a.act, a.act_sc, Gin);
  PairStream<kFp4Depth> st[2];
  st[0].init(up, rb, nkt, Gin, p0, p1, se);
  st[1].init(gate, rb, nkt, Gin, p0, p1, se + 16 * ngmax);
  st[0].issue_scales();
  st[1].issue_scales();
  st[0].start();  // unconditional (an empty range re-reads pair 0): the waits stay exact
  st[1].start();
  FP4_TRACE(1);  // weight streams started
  stage.finish(act_pairs, act_exp);
  st[0].finish_scales();
  st[1].finish_scales();
  __syncthreads();
  FP4_TRACE(2);  // activations and scales staged
  double acc[2] = {0.0, 0.0};
  if (p0 < p1) run_streams<kFp4Depth, 2>(st, act_pairs, act_exp, acc);
  FP4_TRACE(3);  // (wave 0) streams done
  double u = acc[0], g = acc[1];
  u += shfl_xor_d(u, 16);
  g += shfl_xor_d(g, 16);
  u += shfl_xor_d(u, 32);
  g += shfl_xor_d(g, 32);
  if (lane < 16) {
    part[wave][lane][0] = u;
    part[wave][lane][1] = g;
  }
  __syncthreads();
  if (wave == 0) {
    // lane t < 32: row 32q + t = row block 2q + (t >> 4), row t & 15; quarters in order
    const int t = lane & 31, w0 = (t >> 4) * 4;
    double su = 0.0, sg = 0.0;
    for (int k = 0; k < 4; k++) {
      su += part[w0 + k][t & 15][0];
      sg += part[w0 + k][t & 15][1];
    }
    const float h = swiglu_fp4((float)sg, (float)su);
    // E8M0 of the 32 rows (lanes 0..31 and their copies 32..63 give the same maximum)
    float amax = fabsf(h);
#pragma unroll
    for (int m = 1; m < 32; m <<= 1) amax = fmaxf(amax, __shfl_xor(amax, m));
    const uint32_t e = e8m0_of_amax(amax);
    const float inv = amax == 0.0f ? 0.0f : e8m0_inv(e);
    const uint32_t code = e2m1_rne(h * inv);
    const uint32_t hi = (uint32_t)__shfl(code, (lane & 15) + 16);
    if (lane < 16) hcodes[(size_t)q * 16 + lane] = (uint8_t)(code | (hi << 4));
    if (lane == 0) hsc[q] = (uint8_t)e;
    (void)hrow;
  }
  put_record();
  FP4_TRACE(4);
}

// Down of every active expert + weighted accumulate (kernels.cu:5519-5591): workgroup rb =
// output rows [16 rb, 16 rb + 16); wave s = slot s over the whole K_mid; the slots' results
// meet in LDS and out[r] += w_s * d_s[r] in slot order.
__global__ __launch_bounds__(512) void k_fp4_down(Fp4Args a) {
  extern __shared__ uint4 lds[];
  const int Gm = a.M_mid / 32, nkt = a.M_mid / 64, P = nkt / 2;
  uint4* hp = lds;                                        // [n][Gm][4]
  int* he = (int*)(lds + (size_t)a.n * Gm * 4);           // [n][Gm]
  __shared__ float d[kFp4MaxActive][16];
  const int rb = (int)blockIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
  const int lane = lane_id();
  const int s = wave;
  const Fp4Mat dn = s < a.n ? slot_mat(a, s, 2, a.M_out, a.M_mid) : Fp4Mat{nullptr, nullptr};
  const bool use = dn.data && dn.scales;
  Stage<1> stage;  // this workgroup's share of every slot's intermediate: one group per thread
  const int ng = a.n * Gm;
  {
    // thread t stages group t of the flattened [slot][group] list (slot stride mid_stride)
    const int t = min((int)threadIdx.x, ng - 1), sl = t / Gm, gi = t - sl * Gm;
    const uint8_t* hc = a.mid + (size_t)sl * a.mid_stride;
    stage.w[0] = *(const uint4*)(hc + (size_t)gi * 16);
    stage.e[0] = hc[a.M_mid / 2 + gi];
    __builtin_amdgcn_sched_barrier(0);
  }
  PairStream<kFp4Depth> sd[1];
  // the scale and first weight loads go out behind the staging loads, unconditionally (an
  // unusable slot streams one pair of the intermediate buffer instead, never used)
  uint8_t* se = (uint8_t*)(he + (size_t)a.n * Gm) + (size_t)wave * 16 * Gm;
  sd[0].init(use ? dn : Fp4Mat{a.mid, (const uint16_t*)a.mid}, use ? rb : 0, nkt, use ? Gm : 0,
             0, use ? P : 1, se);
  sd[0].issue_scales();
  sd[0].start();
  for (int t = (int)threadIdx.x; t < ng; t += (int)blockDim.x) {
    const int sl = t / Gm, gi = t - sl * Gm;
    uint4 w;
    uint8_t e;
    if (t == (int)threadIdx.x) {
      w = stage.w[0];
      e = stage.e[0];
    } else {
      const uint8_t* hc = a.mid + (size_t)sl * a.mid_stride;
      w = *(const uint4*)(hc + (size_t)gi * 16);
      e = hc[a.M_mid / 2 + gi];
    }
    Stage<1>::put(hp + (size_t)sl * Gm * 4, he + (size_t)sl * Gm, gi, w, e);
  }
  sd[0].finish_scales();
  __syncthreads();
  if (s < a.n) {
    float ds = 0.0f;
    if (use) {
      double acc[1];
      run_streams<kFp4Depth, 1>(sd, hp + (size_t)s * Gm * 4, he + (size_t)s * Gm, acc);
      acc[0] += shfl_xor_d(acc[0], 16);
      acc[0] += shfl_xor_d(acc[0], 32);
      ds = (float)acc[0];
    }
    if (lane < 16) d[s][lane] = ds;
  }
  __syncthreads();
  if (threadIdx.x < 16) {
    const int r = rb * 16 + (int)threadIdx.x;
    float o = a.out[r];
    for (int t = 0; t < a.n; t++) {
      float w;
      if (a.table) {
        const int id = (int)a.ids[t];
        if (id >= a.E || !a.table[((size_t)a.layer * a.E + id) * 3 + 2]) continue;
        w = a.wts_dev[t];
      } else {
        if (!a.mat[t][2].data || !a.mat[t][2].scales) continue;
        w = a.wts[t];
      }
      o = add_mul_rn(o, w, d[t][threadIdx.x]);
    }
    a.out[r] = o;
  }
}

// Sequential -> split-half within every 16-byte block (kernels.cu:4125-4160).
__global__ void k_fp4_split_half(uint8_t* data, long long nblocks) {
  const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= nblocks) return;
  uint4* p = (uint4*)(data + i * 16);
  const uint4 v = *p;
  const uint32_t in[4] = {v.x, v.y, v.z, v.w};
  uint32_t out[4] = {0, 0, 0, 0};
#pragma unroll
  for (int j = 0; j < 8; j++) {
    const uint32_t s0 = (in[j >> 2] >> (8 * (j & 3))) & 0xff;
    const uint32_t s1 = (in[(j + 8) >> 2] >> (8 * ((j + 8) & 3))) & 0xff;
    const uint32_t b0 = (s0 & 0x0f) | ((s1 & 0x0f) << 4);
    const uint32_t b1 = (s0 >> 4) | (s1 & 0xf0);
    out[(2 * j) >> 2] |= b0 << (8 * ((2 * j) & 3));
    out[(2 * j + 1) >> 2] |= b1 << (8 * ((2 * j + 1) & 3));
  }
  *p = make_uint4(out[0], out[1], out[2], out[3]);
}

// Row-major split-half [M][K/2] -> tiled (kernels.cu:4190-4225): one 32-byte row piece per thread.
__global__ void k_fp4_to_tiled(const uint8_t* src, uint8_t* dst, int M, int pk) {
  const int nkt = pk / 32;
  const long long total = (long long)(M / 16) * nkt * 16;
  const long long c = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  if (c >= total) return;
  const int r_in = (int)(c % 16);
  const long long tile = c / 16;
  const int t = (int)(tile % nkt);
  const long long rb = tile / nkt;
  const long long row = rb * 16 + r_in;
  const uint4* s = (const uint4*)(src + row * pk + (long long)t * 32);
  uint4* o = (uint4*)(dst + (rb * nkt + t) * 512 + (long long)r_in * 32);
  o[0] = s[0];
  o[1] = s[1];
}

// ------------------------------------------------------------------------- host side

// Per-device intermediate buffer of the fused layer (h of every slot, FP4 + E8M0), allocated by
// vib3_moe_prewarm_gpu_bufs only: the launches never allocate.
struct MidBuf {
  uint8_t* ptr = nullptr;
  size_t stride = 0;  // bytes per slot
  int max_mid = 0;
};
MidBuf g_mid[64];
std::mutex g_mid_lock;

// per slot: codes, E8M0 bytes, and at the end of the slot's stride the 16-byte down record
size_t mid_stride(int m_mid) {
  return ((size_t)m_mid / 2 + (size_t)m_mid / 32 + kDownRecord + 255) / 256 * 256;
}

int current_device() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return -1;
  return dev;
}

// LDS of the two kernels: decoded activation / intermediate groups (64 + 4 bytes each) plus
// each wave's E8M0 bytes of its block's scales.
size_t gateup_lds(int K_in) {
  const int Gin = K_in / 32, P = K_in / 128;
  return (size_t)Gin * 68 + (size_t)8 * 2 * 16 * (4 * ((P + 3) / 4));
}
size_t down_lds(int n, int M_mid) {
  const int Gm = M_mid / 32;
  return (size_t)n * Gm * 68 + (size_t)n * 16 * Gm;
}

// Shape limits of the fused kernels: tiles of 16 rows x 64 columns taken in 128-column pairs,
// 32-row E8M0 groups of h, each kernel's LDS within 64 KB.
int check_shape(int n, int K_in, int M_mid, int K_mid, int M_out) {
  if (n <= 0 || n > kFp4MaxActive) return VIB3_ERR_BAD_COUNT;  // kernels.cu:5672
  if (K_in <= 0 || M_mid <= 0 || M_out <= 0 || K_mid != M_mid) return VIB3_ERR_BAD_COUNT;
  if (K_in % 128 || M_mid % 128 || M_out % 16) return VIB3_ERR_UNSUPPORTED;
  if (gateup_lds(K_in) > 65536 || down_lds(n, M_mid) > 65536) return VIB3_ERR_UNSUPPORTED;
  return 0;
}

int prewarm(int mid);

// The slots' intermediate buffer: the caller's workspace (the _ws entry points), else the
// device's buffer from vib3_moe_prewarm_gpu_bufs, allocated here on first use when the stream
// is not being captured (as the reference's launchers do, kernels.cu:5675); under capture
// without a prewarm, VIB3_ERR_WORKSPACE.
int bind_mid(Fp4Args& a, hipStream_t st, void* ws, size_t ws_bytes) {
  if (ws) {
    const size_t stride = mid_stride(a.M_mid);
    if (((uintptr_t)ws & 255) || ws_bytes < stride * kFp4MaxActive) return VIB3_ERR_WORKSPACE;
    a.mid = (uint8_t*)ws;
    a.mid_stride = stride;
    return 0;
  }
  const int dev = current_device();
  if (dev < 0) return VIB3_ERR_BAD_POINTER;
  MidBuf mb;
  {
    std::lock_guard<std::mutex> lock(g_mid_lock);
    mb = g_mid[dev];
  }
  if (!mb.ptr || mb.max_mid < a.M_mid) {
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(st, &cs) != hipSuccess || cs != hipStreamCaptureStatusNone)
      return VIB3_ERR_WORKSPACE;
    const int rc = prewarm(a.M_mid);
    if (rc) return rc;
    std::lock_guard<std::mutex> lock(g_mid_lock);
    mb = g_mid[dev];
  }
  a.mid = mb.ptr;
  a.mid_stride = mb.stride;
  return 0;
}

int launch_fused(Fp4Args& a, hipStream_t st, void* ws = nullptr, size_t ws_bytes = 0) {
  const int rc = bind_mid(a, st, ws, ws_bytes);
  if (rc) return rc;
  hipLaunchKernelGGL(k_fp4_gateup, dim3((unsigned)(a.M_mid / 32), (unsigned)a.n), dim3(512),
                     (unsigned)gateup_lds(a.K_in), st, a);
  if (a.M_mid % 512 == 0) {
    // one workgroup per CU, waves owning four output rows each
    const int G4 = a.M_out / 4;
    int wpb = (G4 + device_cus() - 1) / device_cus();
    wpb = wpb < 1 ? 1 : wpb > 16 ? 16 : wpb;
    const dim3 grid((unsigned)((G4 + wpb - 1) / wpb)), block(64 * wpb);
    const unsigned lds = (unsigned)((size_t)a.n * (a.M_mid / 32) * 68);
    if (a.M_mid % 2048 == 0) hipLaunchKernelGGL(k_fp4_down_rows<4>, grid, block, lds, st, a);
    else if (a.M_mid % 1024 == 0) hipLaunchKernelGGL(k_fp4_down_rows<2>, grid, block, lds, st, a);
    else hipLaunchKernelGGL(k_fp4_down_rows<1>, grid, block, lds, st, a);
  } else {
    hipLaunchKernelGGL(k_fp4_down, dim3((unsigned)(a.M_out / 16)), dim3(64 * a.n),
                       (unsigned)down_lds(a.n, a.M_mid), st, a);
  }
  VIB3_RETURN_LAUNCH();
}

int prewarm(int mid) {
  const int dev = current_device();
  if (dev < 0) return VIB3_ERR_BAD_POINTER;
  std::lock_guard<std::mutex> lock(g_mid_lock);
  MidBuf& mb = g_mid[dev];
  if (mb.ptr && mb.max_mid >= mid) return 0;
  const size_t stride = mid_stride(mid);
  void* p = nullptr;
  const hipError_t e = hipMalloc(&p, stride * kFp4MaxActive);
  if (e != hipSuccess) return (int)e;
  // the previous buffer stays allocated: a launch already queued may still read it
  mb.ptr = (uint8_t*)p;
  mb.stride = stride;
  mb.max_mid = mid;
  return 0;
}

}  // namespace
}  // namespace vib3

using namespace vib3;

extern "C" {

int vib3_launch_quantize_activation_fp4(const void* input, void* act_fp4, void* act_scales,
                                        int K, void* stream) {
  if (K <= 0) return VIB3_ERR_BAD_COUNT;
  if (!input || !act_fp4 || !act_scales) return VIB3_ERR_BAD_POINTER;
  if (((uintptr_t)act_fp4 & 15)) return VIB3_ERR_BAD_POINTER;
  const int groups = (K + 31) / 32;
  hipLaunchKernelGGL(k_fp4_quant_act, dim3((unsigned)((groups * 32 + 255) / 256)), dim3(256), 0,
                     (hipStream_t)stream, (const float*)input, (uint8_t*)act_fp4,
                     (uint8_t*)act_scales, K);
  VIB3_RETURN_LAUNCH();
}

int vib3_launch_fused_rms_norm_quantize_fp4(const void* input, const void* norm_weight,
                                            void* act_fp4, void* act_scales, void* opt_f16_out,
                                            int K, float eps, void* stream) {
  if (K <= 0) return VIB3_ERR_BAD_COUNT;
  if (K % 32) return VIB3_ERR_UNSUPPORTED;
  if (!input || !norm_weight || !act_fp4 || !act_scales) return VIB3_ERR_BAD_POINTER;
  hipLaunchKernelGGL(k_fp4_rms_quant, dim3((unsigned)((K + 1023) / 1024)), dim3(256), 0,
                     (hipStream_t)stream, (const float*)input, (const uint16_t*)norm_weight,
                     (uint8_t*)act_fp4, (uint8_t*)act_scales, (uint16_t*)opt_f16_out, K, eps);
  VIB3_RETURN_LAUNCH();
}

int vib3_launch_fp16_to_nvfp4_weight(const void* input, void* out_data, void* out_scales, int M,
                                     int K, void* stream) {
  if (M < 0 || K < 0) return VIB3_ERR_BAD_COUNT;
  if (K % 32) return VIB3_ERR_UNSUPPORTED;  // whole groups per row (kernels.cu:6134)
  if (!input || !out_data || !out_scales) return VIB3_ERR_BAD_POINTER;
  const long long n = (long long)M * K;
  if (n == 0) return 0;
  hipLaunchKernelGGL(k_fp4_weight_quant, dim3((unsigned)((n + 255) / 256)), dim3(256), 0,
                     (hipStream_t)stream, (const uint16_t*)input, (uint8_t*)out_data,
                     (uint16_t*)out_scales, n);
  VIB3_RETURN_LAUNCH();
}

int vib3_launch_quantize_activation_fp4_fast(const void* input, void* act_fp4, void* act_scales,
                                             int K, void* stream) {
  return vib3_launch_quantize_activation_fp4(input, act_fp4, act_scales, K, stream);
}

int vib3_moe_prewarm_gpu_bufs(int m_mid, int k_mid) {
  if (m_mid <= 0 || k_mid <= 0) return VIB3_ERR_BAD_COUNT;
  return prewarm(m_mid > k_mid ? m_mid : k_mid);
}

size_t vib3_moe_experts_fused_workspace_bytes(int m_mid) {
  return m_mid > 0 ? mid_stride(m_mid) * kFp4MaxActive : 0;
}

}  // extern "C"

namespace {

int fused_host(const void* act_fp4, const void* act_scales, const void* const* up_weight_ptrs,
               const void* const* up_scale_ptrs, const void* const* gate_weight_ptrs,
               const void* const* gate_scale_ptrs, const void* const* down_weight_ptrs,
               const void* const* down_scale_ptrs, const float* expert_weights_host,
               int num_experts, int K_in, int M_mid, int K_mid, int M_out, float* layer_output,
               void* ws, size_t ws_bytes, void* stream) {
  const int rc = check_shape(num_experts, K_in, M_mid, K_mid, M_out);
  if (rc) return rc;
  if (!act_fp4 || !act_scales || !up_weight_ptrs || !up_scale_ptrs || !gate_weight_ptrs ||
      !gate_scale_ptrs || !down_weight_ptrs || !down_scale_ptrs || !expert_weights_host ||
      !layer_output)
    return VIB3_ERR_BAD_POINTER;
  Fp4Args a{};
  a.act = (const uint8_t*)act_fp4;
  a.act_sc = (const uint8_t*)act_scales;
  a.n = num_experts;
  a.K_in = K_in; a.M_mid = M_mid; a.M_out = M_out;
  a.out = layer_output;
  for (int s = 0; s < num_experts; s++) {
    a.mat[s][0] = Fp4Mat{(const uint8_t*)up_weight_ptrs[s], (const uint16_t*)up_scale_ptrs[s]};
    a.mat[s][1] = Fp4Mat{(const uint8_t*)gate_weight_ptrs[s], (const uint16_t*)gate_scale_ptrs[s]};
    a.mat[s][2] = Fp4Mat{(const uint8_t*)down_weight_ptrs[s], (const uint16_t*)down_scale_ptrs[s]};
    a.wts[s] = expert_weights_host[s];
  }
  return launch_fused(a, (hipStream_t)stream, ws, ws_bytes);
}

int fused_dev(const void* act_fp4, const void* act_scales, const uint64_t* page_table,
              const uint16_t* expert_ids, const float* expert_weights, int layer,
              int num_experts_total, int num_active, int K_in, int M_mid, int K_mid, int M_out,
              float* layer_output, void* ws, size_t ws_bytes, void* stream) {
  const int rc = check_shape(num_active, K_in, M_mid, K_mid, M_out);
  if (rc) return rc;
  if (layer < 0 || num_experts_total <= 0) return VIB3_ERR_BAD_COUNT;
  if (!act_fp4 || !act_scales || !page_table || !expert_ids || !expert_weights || !layer_output)
    return VIB3_ERR_BAD_POINTER;
  Fp4Args a{};
  a.act = (const uint8_t*)act_fp4;
  a.act_sc = (const uint8_t*)act_scales;
  a.table = page_table;
  a.ids = expert_ids;
  a.wts_dev = expert_weights;
  a.layer = layer;
  a.E = num_experts_total;
  a.n = num_active;
  a.K_in = K_in; a.M_mid = M_mid; a.M_out = M_out;
  a.out = layer_output;
  return launch_fused(a, (hipStream_t)stream, ws, ws_bytes);
}

}  // namespace

extern "C" {

int vib3_launch_moe_experts_fused(const void* act_fp4, const void* act_scales,
                                  const void* const* up_weight_ptrs,
                                  const void* const* up_scale_ptrs,
                                  const void* const* gate_weight_ptrs,
                                  const void* const* gate_scale_ptrs,
                                  const void* const* down_weight_ptrs,
                                  const void* const* down_scale_ptrs,
                                  const float* expert_weights_host, int num_experts, int K_in,
                                  int M_mid, int K_mid, int M_out, float* layer_output,
                                  void* stream) {
  return fused_host(act_fp4, act_scales, up_weight_ptrs, up_scale_ptrs, gate_weight_ptrs,
                    gate_scale_ptrs, down_weight_ptrs, down_scale_ptrs, expert_weights_host,
                    num_experts, K_in, M_mid, K_mid, M_out, layer_output, nullptr, 0, stream);
}

int vib3_launch_moe_experts_fused_ws(const void* act_fp4, const void* act_scales,
                                     const void* const* up_weight_ptrs,
                                     const void* const* up_scale_ptrs,
                                     const void* const* gate_weight_ptrs,
                                     const void* const* gate_scale_ptrs,
                                     const void* const* down_weight_ptrs,
                                     const void* const* down_scale_ptrs,
                                     const float* expert_weights_host, int num_experts, int K_in,
                                     int M_mid, int K_mid, int M_out, float* layer_output,
                                     void* workspace, size_t workspace_bytes, void* stream) {
  if (!workspace) return VIB3_ERR_BAD_POINTER;
  return fused_host(act_fp4, act_scales, up_weight_ptrs, up_scale_ptrs, gate_weight_ptrs,
                    gate_scale_ptrs, down_weight_ptrs, down_scale_ptrs, expert_weights_host,
                    num_experts, K_in, M_mid, K_mid, M_out, layer_output, workspace,
                    workspace_bytes, stream);
}

int vib3_launch_moe_experts_fused_gpu(const void* act_fp4, const void* act_scales,
                                      const uint64_t* page_table, const uint16_t* expert_ids,
                                      const float* expert_weights, int layer,
                                      int num_experts_total, int num_active, int K_in, int M_mid,
                                      int K_mid, int M_out, float* layer_output, void* stream) {
  return fused_dev(act_fp4, act_scales, page_table, expert_ids, expert_weights, layer,
                   num_experts_total, num_active, K_in, M_mid, K_mid, M_out, layer_output,
                   nullptr, 0, stream);
}

int vib3_launch_moe_experts_fused_gpu_ws(const void* act_fp4, const void* act_scales,
                                         const uint64_t* page_table, const uint16_t* expert_ids,
                                         const float* expert_weights, int layer,
                                         int num_experts_total, int num_active, int K_in,
                                         int M_mid, int K_mid, int M_out, float* layer_output,
                                         void* workspace, size_t workspace_bytes, void* stream) {
  if (!workspace) return VIB3_ERR_BAD_POINTER;
  return fused_dev(act_fp4, act_scales, page_table, expert_ids, expert_weights, layer,
                   num_experts_total, num_active, K_in, M_mid, K_mid, M_out, layer_output,
                   workspace, workspace_bytes, stream);
}

int vib3_launch_expert_batched(const void* act_fp4, const void* act_scales,
                               const void* up_weight, const void* up_scales,
                               const void* gate_weight, const void* gate_scales,
                               const void* down_weight, const void* down_scales,
                               float* layer_output, float expert_weight, int K_in, int M_mid,
                               int K_mid, int M_out, void* stream) {
  // kernels.cu:4708: one expert's up, gate, SwiGLU, FP4 quantization of h, down and
  // layer_output += expert_weight * down, over tiled split-half pages; the fused pipeline with
  // one active expert computes exactly that
  const void* up[1] = {up_weight};
  const void* us[1] = {up_scales};
  const void* gt[1] = {gate_weight};
  const void* gs[1] = {gate_scales};
  const void* dn[1] = {down_weight};
  const void* ds[1] = {down_scales};
  if (!up_weight || !up_scales || !gate_weight || !gate_scales || !down_weight || !down_scales)
    return VIB3_ERR_BAD_POINTER;
  return fused_host(act_fp4, act_scales, up, us, gt, gs, dn, ds, &expert_weight, 1, K_in,
                    M_mid, K_mid, M_out, layer_output, nullptr, 0, stream);
}

int vib3_launch_repack_weights_inplace(void* weight_data_ptr, long long weight_data_bytes,
                                       void* stream) {
  if (weight_data_bytes < 0) return VIB3_ERR_BAD_COUNT;
  if (!weight_data_ptr || ((uintptr_t)weight_data_ptr & 15)) return VIB3_ERR_BAD_POINTER;
  const long long nblocks = weight_data_bytes / 16;  // a partial last block is left as it is
  if (nblocks == 0) return 0;
  hipLaunchKernelGGL(k_fp4_split_half, dim3((unsigned)((nblocks + 255) / 256)), dim3(256), 0,
                     (hipStream_t)stream, (uint8_t*)weight_data_ptr, nblocks);
  VIB3_RETURN_LAUNCH();
}

int vib3_launch_repack_row_to_tiled(void* weight_data_ptr, void* temp_buf, int M, int K,
                                    void* stream) {
  if (M < 0 || K < 0) return VIB3_ERR_BAD_COUNT;
  if (M % 16 || K % 64) return VIB3_ERR_UNSUPPORTED;  // kernels.cu:4198
  if (!weight_data_ptr || !temp_buf || ((uintptr_t)weight_data_ptr & 15) ||
      ((uintptr_t)temp_buf & 15))
    return VIB3_ERR_BAD_POINTER;
  const int pk = K / 2;
  const long long chunks = (long long)(M / 16) * (pk / 32) * 16;
  if (chunks == 0) return 0;
  hipStream_t st = (hipStream_t)stream;
  hipLaunchKernelGGL(k_fp4_to_tiled, dim3((unsigned)((chunks + 255) / 256)), dim3(256), 0, st,
                     (const uint8_t*)weight_data_ptr, (uint8_t*)temp_buf, M, pk);
  const hipError_t e = hipMemcpyAsync(weight_data_ptr, temp_buf, (size_t)M * pk,
                                      hipMemcpyDeviceToDevice, st);
  if (e != hipSuccess) return (int)e;
  VIB3_RETURN_LAUNCH();
}

}  // extern "C"

#ifdef VIB3_TRACE
// Profiling builds only: where this translation unit's kernels write their timeline probes.
extern "C" int vib3_trace_set_fp4(void* buf) {
  uint64_t* p = (uint64_t*)buf;
  return (int)hipMemcpyToSymbol(HIP_SYMBOL(vib3_trace_buf), &p, sizeof(p));
}
#endif
