// fp4_pages.hip — the reference's per-page NVFP4 launchers, the path execute_expert takes for
// NVFP4 experts that do not fit the fused table's one page per segment (engine.rs:5960-6226):
//
//   block-scaled GEMV (E2M1 weights x FP4-quantized activation, E8M0 scales):
//     vib3_launch_gemv_mma_nvfp4_preq[_fast]          kernels.cu:3752, :5229  row-major split-half
//     vib3_launch_fused_swiglu_mma_nvfp4_preq[_fast]  kernels.cu:3853, :5267  (SwiGLU of two)
//     vib3_launch_gemv_mma_nvfp4_tiled                kernels.cu:4359         tiled split-half
//     vib3_launch_gemv_scalar_nvfp4                   kernels.cu:4520         full bf16 scales
//     vib3_launch_gemv_mma_nvfp4, _fused_swiglu_mma_nvfp4  kernels.cu:3676, :3807  f32 input,
//                                                     quantized in the kernel; sequential codes
//   f32 GEMV over dequantized weights (the reference's scalar kernels, no activation rounding):
//     vib3_launch_partial_matmul_nvfp4[_f32out|_fp16in]  kernels.cu:1524, :2499, :1552
//     vib3_launch_fused_swiglu_nvfp4[_f32out]            kernels.cu:1537, :2483
//
// Layouts: a page is [rows][K/2] code bytes, then [rows][K/32] 2-byte scales (kernels.rs:
// 821-860: scales at page + K/2 * rows). "Sequential" bytes hold values 2j (low nibble) and
// 2j + 1; "split-half" 16-byte groups hold values j and j + 16 (after
// vib3_launch_repack_weights_inplace); "tiled" puts 16 rows x 64 values in 512-byte tiles
// (after vib3_launch_repack_row_to_tiled). The block-scaled kernels read a scale's exponent
// byte as E8M0, like the MMA instruction (kernels.cu:3355); the scalar ones its bf16 value.
//
// Arithmetic of the block-scaled kernels: as in fp4_fused.hip, each 32-value group's dot
// product is exact in f32, scaled by exact powers of two and summed in f64, the row rounded to
// f32 once: the result does not depend on the summation order and equals the oracle's. The
// scalar kernels accumulate x * w * s in f32 (an order of their own, as the reference's warp
// reductions have theirs).
#include "common.h"
#include "fp4.h"
#include "kernels.h"

namespace vib3 {
namespace {

enum { kLayRowSplit = 0, kLayTiled = 1, kLaySeq = 2 };

struct PageGemvArgs {
  const uint8_t* act;     // split-half activation codes [K/32][16], or null: quantize x
  const uint8_t* act_sc;  // [K/32] E8M0
  const float* x;         // f32 activation when act is null
  const uint8_t* w[2];    // code bytes of one matrix, or up and gate
  const uint16_t* s[2];   // their scales [M][K/32]
  float* out;             // [M] f32
  int K, M;
};

// Sequential 16 bytes (value 2j low, 2j + 1 high) as split-half (byte j: value j | value j + 16).
__device__ __forceinline__ uint4 seq_to_split(uint4 v) {
  const uint32_t in[4] = {v.x, v.y, v.z, v.w};
  uint32_t o[4] = {0, 0, 0, 0};
#pragma unroll
  for (int j = 0; j < 8; j++) {
    const uint32_t s0 = (in[j >> 2] >> (8 * (j & 3))) & 0xff;
    const uint32_t s1 = (in[(j + 8) >> 2] >> (8 * ((j + 8) & 3))) & 0xff;
    o[(2 * j) >> 2] |= ((s0 & 0x0f) | ((s1 & 0x0f) << 4)) << (8 * ((2 * j) & 3));
    o[(2 * j + 1) >> 2] |= ((s0 >> 4) | (s1 & 0xf0)) << (8 * ((2 * j + 1) & 3));
  }
  return make_uint4(o[0], o[1], o[2], o[3]);
}

// One group's 16 split-half bytes as the LDS pair layout group_dot reads.
__device__ __forceinline__ void put_group(uint4* pairs, int* ex, int g, uint4 w, int e) {
  f16x2 p[16];
  decode_group(w, p);
#pragma unroll
  for (int q = 0; q < 4; q++)
    pairs[(size_t)g * 4 + q] =
        make_uint4(__builtin_bit_cast(uint32_t, p[4 * q]), __builtin_bit_cast(uint32_t, p[4 * q + 1]),
                   __builtin_bit_cast(uint32_t, p[4 * q + 2]), __builtin_bit_cast(uint32_t, p[4 * q + 3]));
  ex[g] = e;
}

// Bytes of group g of row r in layout LAY.
template <int LAY>
__device__ __forceinline__ const uint8_t* group_ptr(const uint8_t* w, int r, int g, int K) {
  if (LAY == kLayTiled)
    return w + ((size_t)(r >> 4) * (K / 64) + (g >> 1)) * 512 + (r & 15) * 32 + (g & 1) * 16;
  return w + (size_t)r * (K / 2) + (size_t)g * 16;
}

// Workgroup = 16 rows, 16 lanes per row (a lane takes groups l, l + 16, ...), the activation
// staged once per workgroup in LDS as decoded pairs and exponents.
template <int LAY, bool FULL, int NS>
__global__ __launch_bounds__(256) void k_fp4_page_gemv(PageGemvArgs a) {
  extern __shared__ uint4 lds[];
  const int G = a.K / 32, tid = (int)threadIdx.x, lane = lane_id();
  uint4* pairs = lds;                      // [G][4]
  int* ex = (int*)(lds + (size_t)G * 4);   // [G]
  if (a.act) {
    for (int g = tid; g < G; g += 256) put_group(pairs, ex, g, *(const uint4*)(a.act + (size_t)g * 16), a.act_sc[g]);
  } else {
    // the activation quantizer's rule (kernels.cu:3193-3240, inline at :3418-3470): a 32-lane
    // half-wave per group, E8M0 of its absolute maximum, codes rounded to nearest even
    uint8_t* codes = (uint8_t*)(ex + G);  // [G][16]
    int* es = (int*)(codes + (size_t)G * 16 + 16);
    es = (int*)(((uintptr_t)es + 3) & ~(uintptr_t)3);
    for (int base = 0; base < G * 32; base += 256) {
      const int i = base + tid;
      const float v = i < a.K ? a.x[i] : 0.0f;
      float amax = fabsf(v);
#pragma unroll
      for (int m = 1; m < 32; m <<= 1) amax = fmaxf(amax, __shfl_xor(amax, m));
      const uint32_t e = e8m0_of_amax(amax);
      const float inv = amax == 0.0f ? 0.0f : e8m0_inv(e);
      const uint32_t code = e2m1_rne(v * inv);
      const uint32_t hi = (uint32_t)__shfl(code, (lane & ~31) + (lane & 15) + 16);
      const int g = i >> 5, j = i & 31;
      if (j < 16 && g < G) codes[(size_t)g * 16 + j] = (uint8_t)(code | (hi << 4));
      if (j == 0 && g < G) es[g] = (int)e;
    }
    __syncthreads();
    for (int g = tid; g < G; g += 256) put_group(pairs, ex, g, *(const uint4*)(codes + (size_t)g * 16), es[g]);
  }
  __syncthreads();
  const int gl = tid & 15, row = (int)blockIdx.x * 16 + (tid >> 4);
  const int rc = row < a.M ? row : a.M - 1;
  double acc[NS];
#pragma unroll
  for (int m = 0; m < NS; m++) acc[m] = 0.0;
  for (int g = gl; g < G; g += 16) {
    const double ea = pow2d(ex[g] - 127);
#pragma unroll
    for (int m = 0; m < NS; m++) {
      uint4 w = *(const uint4*)group_ptr<LAY>(a.w[m], rc, g, a.K);
      if (LAY == kLaySeq) w = seq_to_split(w);
      const uint16_t sw = a.s[m][(size_t)rc * G + g];
      const double ws = FULL ? (double)bf16_to_f32(sw) : pow2d((int)((sw >> 7) & 0xff) - 127);
      acc[m] = fma((double)group_dot(w, pairs + (size_t)g * 4), ws * ea, acc[m]);
    }
  }
#pragma unroll
  for (int m = 0; m < NS; m++)
#pragma unroll
    for (int o = 1; o < 16; o <<= 1) acc[m] += shfl_xor_d(acc[m], o);
  if (gl == 0 && row < a.M)
    a.out[row] = NS == 1 ? (float)acc[0] : swiglu_fp4((float)acc[1], (float)acc[0]);
}

struct ScalarArgs {
  const void* x;          // f32 or f16 [K]
  const uint8_t* w[2];    // sequential codes [M][K/2]
  const uint16_t* s[2];   // bf16 scales [M][K / bs]
  void* out;              // f16 or f32 [M]
  int K, M, bs_shift;     // block size 32 << bs_shift... as a shift of 32-value groups
};

__device__ __forceinline__ float e2m1_lut(uint32_t q) {
  const float m[8] = {0.0f, 0.5f, 1.0f, 1.5f, 2.0f, 3.0f, 4.0f, 6.0f};
  const float v = m[q & 7];
  return (q & 8) ? -v : v;
}

// out[r] = sum_k x[k] * e2m1(W[r][k]) * bf16(s[r][k / bs]) in f32: per 32-value group the
// products x * e2m1 summed with fused multiply-adds, then times the block scale into the row
// sum; SwiGLU (NS = 2: up, gate) as the reference's epilogue silu(g) * u with
// silu(g) = g / (1 + e^-g) (kernels.cu:580-582, :2027-2028). x staged in LDS as f32.
template <bool IN16, bool OUT16, int NS>
__global__ __launch_bounds__(256) void k_nvfp4_scalar(ScalarArgs a) {
  extern __shared__ float xs[];
  const int tid = (int)threadIdx.x, G = a.K / 32;
  for (int i = tid; i < a.K; i += 256)
    xs[i] = IN16 ? f16_to_f32(((const uint16_t*)a.x)[i]) : ((const float*)a.x)[i];
  __syncthreads();
  const int gl = tid & 15, row = (int)blockIdx.x * 16 + (tid >> 4);
  const int rc = row < a.M ? row : a.M - 1;
  const int nb = G >> a.bs_shift;
  float acc[NS];
#pragma unroll
  for (int m = 0; m < NS; m++) acc[m] = 0.0f;
  for (int g = gl; g < G; g += 16) {
#pragma unroll
    for (int m = 0; m < NS; m++) {
      const uint4 w = *(const uint4*)(a.w[m] + (size_t)rc * (a.K / 2) + (size_t)g * 16);
      const uint32_t wd[4] = {w.x, w.y, w.z, w.w};
      float p = 0.0f;
#pragma unroll
      for (int i = 0; i < 16; i++) {
        const uint32_t b = (wd[i >> 2] >> (8 * (i & 3))) & 0xff;
        p = __builtin_fmaf(xs[g * 32 + 2 * i], e2m1_lut(b & 15), p);
        p = __builtin_fmaf(xs[g * 32 + 2 * i + 1], e2m1_lut(b >> 4), p);
      }
      acc[m] = __builtin_fmaf(p, bf16_to_f32(a.s[m][(size_t)rc * nb + (g >> a.bs_shift)]), acc[m]);
    }
  }
#pragma unroll
  for (int m = 0; m < NS; m++)
#pragma unroll
    for (int o = 1; o < 16; o <<= 1) acc[m] += __shfl_xor(acc[m], o);
  if (gl == 0 && row < a.M) {
    float v = acc[0];
    if (NS == 2) v = (acc[1] / (1.0f + expf(-acc[1]))) * acc[0];
    if (OUT16) ((uint16_t*)a.out)[row] = f32_to_f16_bits(v);
    else ((float*)a.out)[row] = v;
  }
}

int page_gemv(int lay, bool full, int ns, const void* act, const void* act_sc, const float* x,
              const void* w0, const void* s0, const void* w1, const void* s1, void* out, int K,
              int M, void* stream) {
  if (K <= 0 || M < 0) return VIB3_ERR_BAD_COUNT;
  if (K % 32 || (lay == kLayTiled && (K % 64 || M % 16))) return VIB3_ERR_UNSUPPORTED;
  if ((!act && !x) || (act && !act_sc) || !w0 || !s0 || !out || (ns == 2 && (!w1 || !s1)))
    return VIB3_ERR_BAD_POINTER;
  if ((((uintptr_t)w0 | (uintptr_t)(ns == 2 ? w1 : w0) | (uintptr_t)(act ? act : w0)) & 15))
    return VIB3_ERR_BAD_POINTER;
  if (M == 0) return 0;
  const int G = K / 32;
  const size_t lds = (size_t)G * 68 + (act ? 0 : (size_t)G * 20 + 32);
  if (lds > 65536) return VIB3_ERR_UNSUPPORTED;
  PageGemvArgs a{};
  a.act = (const uint8_t*)act; a.act_sc = (const uint8_t*)act_sc; a.x = x;
  a.w[0] = (const uint8_t*)w0; a.s[0] = (const uint16_t*)s0;
  a.w[1] = (const uint8_t*)w1; a.s[1] = (const uint16_t*)s1;
  a.out = (float*)out; a.K = K; a.M = M;
  const dim3 grid((unsigned)((M + 15) / 16)), block(256);
  hipStream_t st = (hipStream_t)stream;
#define VIB3_PAGE_GEMV(L, F, N) hipLaunchKernelGGL((k_fp4_page_gemv<L, F, N>), grid, block, (unsigned)lds, st, a)
  if (lay == kLayRowSplit && !full && ns == 1) VIB3_PAGE_GEMV(kLayRowSplit, false, 1);
  else if (lay == kLayRowSplit && !full && ns == 2) VIB3_PAGE_GEMV(kLayRowSplit, false, 2);
  else if (lay == kLayRowSplit && full && ns == 1) VIB3_PAGE_GEMV(kLayRowSplit, true, 1);
  else if (lay == kLayTiled && !full && ns == 1) VIB3_PAGE_GEMV(kLayTiled, false, 1);
  else if (lay == kLaySeq && !full && ns == 1) VIB3_PAGE_GEMV(kLaySeq, false, 1);
  else if (lay == kLaySeq && !full && ns == 2) VIB3_PAGE_GEMV(kLaySeq, false, 2);
  else return VIB3_ERR_UNSUPPORTED;
#undef VIB3_PAGE_GEMV
  VIB3_RETURN_LAUNCH();
}

int scalar_gemv(bool in16, bool out16, int ns, const void* x, const void* w0, const void* s0,
                const void* w1, const void* s1, void* out, int K, int M, int bs, void* stream) {
  if (K <= 0 || M < 0 || bs <= 0) return VIB3_ERR_BAD_COUNT;
  if (K % 32 || bs % 32 || (bs & (bs - 1)) || (K / 32) % (bs / 32)) return VIB3_ERR_UNSUPPORTED;
  if ((size_t)K * 4 > 65536) return VIB3_ERR_UNSUPPORTED;
  if (!x || !w0 || !s0 || !out || (ns == 2 && (!w1 || !s1))) return VIB3_ERR_BAD_POINTER;
  if ((((uintptr_t)w0 | (uintptr_t)(ns == 2 ? w1 : w0)) & 15)) return VIB3_ERR_BAD_POINTER;
  if (M == 0) return 0;
  ScalarArgs a{};
  a.x = x; a.w[0] = (const uint8_t*)w0; a.s[0] = (const uint16_t*)s0;
  a.w[1] = (const uint8_t*)w1; a.s[1] = (const uint16_t*)s1;
  a.out = out; a.K = K; a.M = M; a.bs_shift = __builtin_ctz((unsigned)(bs / 32));
  const dim3 grid((unsigned)((M + 15) / 16)), block(256);
  const unsigned lds = (unsigned)K * 4;
  hipStream_t st = (hipStream_t)stream;
  if (!in16 && out16 && ns == 1) hipLaunchKernelGGL((k_nvfp4_scalar<false, true, 1>), grid, block, lds, st, a);
  else if (!in16 && !out16 && ns == 1) hipLaunchKernelGGL((k_nvfp4_scalar<false, false, 1>), grid, block, lds, st, a);
  else if (in16 && out16 && ns == 1) hipLaunchKernelGGL((k_nvfp4_scalar<true, true, 1>), grid, block, lds, st, a);
  else if (!in16 && out16 && ns == 2) hipLaunchKernelGGL((k_nvfp4_scalar<false, true, 2>), grid, block, lds, st, a);
  else if (!in16 && !out16 && ns == 2) hipLaunchKernelGGL((k_nvfp4_scalar<false, false, 2>), grid, block, lds, st, a);
  else return VIB3_ERR_UNSUPPORTED;
  VIB3_RETURN_LAUNCH();
}

}  // namespace
}  // namespace vib3

using namespace vib3;

extern "C" {

int vib3_launch_gemv_mma_nvfp4_preq(const void* act_fp4, const void* act_scales,
                                    const void* weight_packed, const void* scales, void* output,
                                    int K, int M_slice, void* stream) {
  return page_gemv(kLayRowSplit, false, 1, act_fp4, act_scales, nullptr, weight_packed, scales,
                   nullptr, nullptr, output, K, M_slice, stream);
}

int vib3_launch_gemv_mma_nvfp4_preq_fast(const void* act_fp4, const void* act_scales,
                                         const void* weight_packed, const void* scales,
                                         void* output, int K, int M_slice, void* stream) {
  return vib3_launch_gemv_mma_nvfp4_preq(act_fp4, act_scales, weight_packed, scales, output, K,
                                         M_slice, stream);
}

int vib3_launch_fused_swiglu_mma_nvfp4_preq(const void* act_fp4, const void* act_scales,
                                            const void* up_weight, const void* up_scales,
                                            const void* gate_weight, const void* gate_scales,
                                            void* output, int K, int M_slice, void* stream) {
  return page_gemv(kLayRowSplit, false, 2, act_fp4, act_scales, nullptr, up_weight, up_scales,
                   gate_weight, gate_scales, output, K, M_slice, stream);
}

int vib3_launch_fused_swiglu_mma_nvfp4_preq_fast(const void* act_fp4, const void* act_scales,
                                                 const void* up_weight, const void* up_scales,
                                                 const void* gate_weight, const void* gate_scales,
                                                 void* output, int K, int M_slice, void* stream) {
  return vib3_launch_fused_swiglu_mma_nvfp4_preq(act_fp4, act_scales, up_weight, up_scales,
                                                 gate_weight, gate_scales, output, K, M_slice,
                                                 stream);
}

int vib3_launch_gemv_mma_nvfp4_tiled(const void* act_fp4, const void* act_scales,
                                     const void* weight, const void* scales, void* output, int K,
                                     int M_slice, void* stream) {
  return page_gemv(kLayTiled, false, 1, act_fp4, act_scales, nullptr, weight, scales, nullptr,
                   nullptr, output, K, M_slice, stream);
}

int vib3_launch_gemv_scalar_nvfp4(const void* act_fp4, const void* act_scales,
                                  const void* weight_packed, const void* scales, void* output,
                                  int K, int M_slice, void* stream) {
  return page_gemv(kLayRowSplit, true, 1, act_fp4, act_scales, nullptr, weight_packed, scales,
                   nullptr, nullptr, output, K, M_slice, stream);
}

int vib3_launch_gemv_mma_nvfp4(const void* input, const void* weight_packed, const void* scales,
                               void* output, int K, int M_slice, void* stream) {
  return page_gemv(kLaySeq, false, 1, nullptr, nullptr, (const float*)input, weight_packed,
                   scales, nullptr, nullptr, output, K, M_slice, stream);
}

int vib3_launch_fused_swiglu_mma_nvfp4(const void* input, const void* up_weight,
                                       const void* up_scales, const void* gate_weight,
                                       const void* gate_scales, void* output, int K,
                                       int M_slice, void* stream) {
  return page_gemv(kLaySeq, false, 2, nullptr, nullptr, (const float*)input, up_weight,
                   up_scales, gate_weight, gate_scales, output, K, M_slice, stream);
}

int vib3_launch_partial_matmul_nvfp4(const void* input, const void* weight_packed,
                                     const void* scales, void* output, int K, int M_slice,
                                     int block_size, void* stream) {
  return scalar_gemv(false, true, 1, input, weight_packed, scales, nullptr, nullptr, output, K,
                     M_slice, block_size, stream);
}

int vib3_launch_partial_matmul_nvfp4_f32out(const void* input, const void* weight_packed,
                                            const void* scales, void* output, int K, int M_slice,
                                            int block_size, void* stream) {
  return scalar_gemv(false, false, 1, input, weight_packed, scales, nullptr, nullptr, output, K,
                     M_slice, block_size, stream);
}

int vib3_launch_partial_matmul_nvfp4_fp16in(const void* input, const void* weight_packed,
                                            const void* scales, void* output, int K, int M_slice,
                                            int block_size, void* stream) {
  return scalar_gemv(true, true, 1, input, weight_packed, scales, nullptr, nullptr, output, K,
                     M_slice, block_size, stream);
}

int vib3_launch_fused_swiglu_nvfp4(const void* input, const void* up_weight,
                                   const void* up_scales, const void* gate_weight,
                                   const void* gate_scales, void* output, int K, int M_slice,
                                   int block_size, void* stream) {
  return scalar_gemv(false, true, 2, input, up_weight, up_scales, gate_weight, gate_scales,
                     output, K, M_slice, block_size, stream);
}

int vib3_launch_fused_swiglu_nvfp4_f32out(const void* input, const void* up_weight,
                                          const void* up_scales, const void* gate_weight,
                                          const void* gate_scales, void* output, int K,
                                          int M_slice, int block_size, void* stream) {
  return scalar_gemv(false, false, 2, input, up_weight, up_scales, gate_weight, gate_scales,
                     output, K, M_slice, block_size, stream);
}

}  // extern "C"
