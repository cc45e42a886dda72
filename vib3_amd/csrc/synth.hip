// synth.hip — on-device synthetic weights and activations (no reference counterpart).
//
// Counter-based, so any slice of any matrix can be regenerated independently and the CPU
// oracle (a separate C implementation of the same spec) produces identical bytes:
//   hash(seed, stream, ctr) = mix(mix(seed ^ stream*C1 + (ctr+1)*C2) + C2), mix = splitmix64
//   normal = (sum of the four 16-bit fields of hash - 131070) * 2.6429e-5f   (Irwin-Hall(4))
//   bytes: byte j = hash(seed, stream, j/8) >> 8*(j%8)
//   scale: |normal(idx + t*2^40)| * sigma rounded to bf16/f16, first t that is non-zero.
// Only exactly-rounded IEEE operations are used (no fused multiply-add), so host and device
// agree bit for bit.
#include "common.h"

namespace vib3 {

__device__ __forceinline__ uint64_t mix64(uint64_t z) {
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

__device__ __forceinline__ uint64_t synth_hash(uint64_t seed, uint64_t stream, uint64_t ctr) {
  uint64_t z = seed ^ (stream * 0xD1B54A32D192ED03ull);
  z += (ctr + 1ull) * 0x9E3779B97F4A7C15ull;
  z = mix64(z);
  return mix64(z + 0x9E3779B97F4A7C15ull);
}

__device__ __forceinline__ float synth_normal(uint64_t seed, uint64_t stream, uint64_t ctr) {
  const uint64_t h = synth_hash(seed, stream, ctr);
  const int32_t s = (int32_t)(h & 0xffff) + (int32_t)((h >> 16) & 0xffff) +
                    (int32_t)((h >> 32) & 0xffff) + (int32_t)(h >> 48) - 131070;
  return __fmul_rn((float)s, 2.6429e-5f);
}

__device__ __forceinline__ uint16_t round_bits(float v, int dt) {
  return dt == VIB3_DT_F16 ? f32_to_f16_bits(v) : f32_to_bf16_bits(v);
}

__device__ __forceinline__ uint16_t synth_scale(uint64_t seed, uint64_t stream, uint64_t idx,
                                                float sigma, int dt) {
  for (uint64_t t = 0;; t++) {
    const float v = __fmul_rn(__builtin_fabsf(synth_normal(seed, stream, idx + (t << 40))), sigma);
    const uint16_t b = round_bits(v, dt);
    if ((b & 0x7fff) != 0) return b;
  }
}

// 8 output bytes per thread; fast path when the logical offset is 8-aligned.
__global__ void k_synth_bytes(uint8_t* dst, size_t n, uint64_t seed, uint64_t stream, size_t off) {
  const size_t t = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  const size_t i0 = t * 8;
  if (i0 >= n) return;
  if ((off & 7) == 0 && i0 + 8 <= n && (((uintptr_t)(dst + i0)) & 7) == 0) {
    *(uint64_t*)(dst + i0) = synth_hash(seed, stream, (off + i0) >> 3);
    return;
  }
  for (size_t i = i0; i < i0 + 8 && i < n; i++) {
    const size_t j = off + i;
    dst[i] = (uint8_t)(synth_hash(seed, stream, j >> 3) >> (8 * (j & 7)));
  }
}

__global__ void k_synth_normal(void* dst, int dt, size_t n, uint64_t seed, uint64_t stream,
                               size_t off, float sigma) {
  const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const float v = __fmul_rn(synth_normal(seed, stream, off + i), sigma);
  if (dt == VIB3_DT_F32) ((float*)dst)[i] = v;
  else ((uint16_t*)dst)[i] = round_bits(v, dt);
}

__global__ void k_synth_scales(uint16_t* dst, size_t n, uint64_t seed, uint64_t stream,
                               size_t off, float sigma, int dt) {
  const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  dst[i] = synth_scale(seed, stream, off + i, sigma, dt);
}

// E8M0 scale bytes 119 + hash % 5: 2^-8 .. 2^-4 (uniform exponent, no zero or NaN codes).
__global__ void k_synth_e8m0(uint8_t* dst, size_t n, uint64_t seed, uint64_t stream, size_t off) {
  const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  dst[i] = (uint8_t)(119 + synth_hash(seed, stream, off + i) % 5);
}

static unsigned blocks_for(size_t n, size_t per_thread) {
  return (unsigned)((n + 256 * per_thread - 1) / (256 * per_thread));
}

}  // namespace vib3

using namespace vib3;

extern "C" {

int vib3_synth_bytes(void* dst, size_t n, uint64_t seed, uint64_t stream, size_t off,
                     void* hip_stream) {
  if (!dst) return VIB3_ERR_BAD_POINTER;
  if (n == 0) return 0;
  hipLaunchKernelGGL(k_synth_bytes, dim3(blocks_for(n, 8)), dim3(256), 0,
                     (hipStream_t)hip_stream, (uint8_t*)dst, n, seed, stream, off);
  VIB3_RETURN_LAUNCH();
}

int vib3_synth_normal(void* dst, int dtype, size_t n, uint64_t seed, uint64_t stream, size_t off,
                      float sigma, void* hip_stream) {
  if (!dst) return VIB3_ERR_BAD_POINTER;
  if (dtype != VIB3_DT_F32 && dtype != VIB3_DT_F16 && dtype != VIB3_DT_BF16)
    return VIB3_ERR_UNSUPPORTED;
  if (n == 0) return 0;
  hipLaunchKernelGGL(k_synth_normal, dim3(blocks_for(n, 1)), dim3(256), 0,
                     (hipStream_t)hip_stream, dst, dtype, n, seed, stream, off, sigma);
  VIB3_RETURN_LAUNCH();
}

int vib3_synth_int4_page(void* page, uint64_t seed, uint64_t stream, int k, int group_size,
                         int scale_dtype, float sigma, int row_start, int rows,
                         void* hip_stream) {
  if (!page) return VIB3_ERR_BAD_POINTER;
  if (k <= 0 || group_size <= 0 || row_start < 0 || rows < 0) return VIB3_ERR_BAD_COUNT;
  if (scale_dtype != VIB3_DT_F16 && scale_dtype != VIB3_DT_BF16) return VIB3_ERR_UNSUPPORTED;
  if (rows == 0) return 0;
  const size_t pk = (size_t)(k + 1) / 2, ng = (size_t)(k + group_size - 1) / group_size;
  hipStream_t s = (hipStream_t)hip_stream;
  const size_t nd = (size_t)rows * pk;
  if (nd % 2) return VIB3_ERR_UNSUPPORTED;  // the scale rows must stay 2-byte aligned
  hipLaunchKernelGGL(k_synth_bytes, dim3(blocks_for(nd, 8)), dim3(256), 0, s, (uint8_t*)page, nd,
                     seed, stream * 2, (size_t)row_start * pk);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return (int)e;
  const size_t ns = (size_t)rows * ng;
  hipLaunchKernelGGL(k_synth_scales, dim3(blocks_for(ns, 1)), dim3(256), 0, s,
                     (uint16_t*)((uint8_t*)page + nd), ns, seed, stream * 2 + 1,
                     (size_t)row_start * ng, sigma, scale_dtype);
  VIB3_RETURN_LAUNCH();
}

int vib3_synth_mxfp4_page(void* page, uint64_t seed, uint64_t stream, int k, int row_start,
                          int rows, void* hip_stream) {
  if (!page) return VIB3_ERR_BAD_POINTER;
  if (k <= 0 || k % 32 || row_start < 0 || rows < 0) return VIB3_ERR_BAD_COUNT;
  if (rows == 0) return 0;
  hipStream_t s = (hipStream_t)hip_stream;
  const size_t pk = (size_t)k / 2, nb = (size_t)k / 32;
  const size_t nd = (size_t)rows * pk;
  hipLaunchKernelGGL(k_synth_bytes, dim3(blocks_for(nd, 8)), dim3(256), 0, s, (uint8_t*)page, nd,
                     seed, stream * 2, (size_t)row_start * pk);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return (int)e;
  const size_t ns = (size_t)rows * nb;
  hipLaunchKernelGGL(k_synth_e8m0, dim3(blocks_for(ns, 1)), dim3(256), 0, s,
                     (uint8_t*)page + nd, ns, seed, stream * 2 + 1, (size_t)row_start * nb);
  VIB3_RETURN_LAUNCH();
}

}  // extern "C"
