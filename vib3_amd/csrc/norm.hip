// norm.hip — the operations either side of the MoE sublayer in vib3's decode step
// (engine.rs:5064-5110 pre-MoE RMSNorm, :5300-5307 residual add, :6392-6425 shared-expert
// sigmoid gate), as standalone launchers with the reference's C ABI and as the prologue of the
// fused layer.
//
// RMSNorm follows vib3_rms_norm_f32 (kernels.cu:921-955): thread t of 256 accumulates x[d]^2
// for d = t, t + 256, ... with fused multiply-adds (the CUDA compiler contracts
// `partial_ss += val * val`), the 256 partials are summed by a halving tree, then
// rms = sqrt(ss / D + eps), inv = 1 / rms (both correctly rounded) and
// y[d] = (x[d] * inv) * w[d] with two rounded products. Every workgroup of a launch computes
// the same inverse RMS in that order, so a launch can spread the output over many workgroups
// and still produce the single-workgroup reference result bit for bit.
#include "common.h"
#include "kernels.h"

namespace vib3 {

// Inverse RMS of x[0..D) for a 256-thread workgroup, in the reference's summation order.
__device__ float wg_inv_rms(const float* x, int D, float eps) {
  __shared__ float ss[256];
  const int tid = (int)threadIdx.x;
  float p = 0.0f;
  for (int d = tid; d < D; d += 256) {
    const float v = x[d];
    p = __builtin_fmaf(v, v, p);
  }
  ss[tid] = p;
  __syncthreads();
  for (int s = 128; s > 0; s >>= 1) {
    if (tid < s) ss[tid] += ss[tid + s];
    __syncthreads();
  }
  const float rms = sqrtf(ss[0] / (float)D + eps);
  const float inv = 1.0f / rms;
  __syncthreads();  // ss is reused by the caller's next call
  return inv;
}

__device__ __forceinline__ float norm_elem(float x, float inv, uint16_t w) {
#pragma clang fp contract(off)
  return x * inv * f16_to_f32(w);
}

// RMSNorm of an f32 vector with f16 weights; OUT_F16 rounds the result to f16. Workgroup b
// writes elements [b * 1024, (b + 1) * 1024).
template <bool OUT_F16>
__global__ __launch_bounds__(256) void k_rms_norm(const float* x, void* out, const uint16_t* w,
                                                 int D, float eps) {
  const float inv = wg_inv_rms(x, D, eps);
  const int d0 = (int)blockIdx.x * 1024;
  for (int d = d0 + (int)threadIdx.x; d < min(D, d0 + 1024); d += 256) {
    const float y = norm_elem(x[d], inv, w[d]);
    if (OUT_F16)
      ((uint16_t*)out)[d] = f32_to_f16_bits(y);
    else
      ((float*)out)[d] = y;
  }
}

// accumulator[i] += layer_output[i] (kernels.cu:817).
__global__ void k_residual_add(float* acc, const float* lo, int n) {
  const int i = (int)(blockIdx.x * blockDim.x + threadIdx.x);
  if (i < n) acc[i] = acc[i] + lo[i];
}

// output[i] += sigmoid(gate[0]) * f32(expert_output[i]) (kernels.cu:2106), with the product
// rounded before the add like the layer's other expert sums.
__global__ void k_sigmoid_gated_acc(float* out, const uint16_t* e, const float* gate, int n) {
  const float g = gate[0];
  const float sg = 1.0f / (1.0f + expf(-g));
  const int i = (int)(blockIdx.x * blockDim.x + threadIdx.x);
  if (i < n) out[i] = add_mul_rn(out[i], sg, f16_to_f32(e[i]));
}

// Prologue of the fused layer. Workgroups [0, nblk) write the normalised activation
// xn = RMSNorm(x) (f32, as engine.rs's moe_normed_f32) when a norm weight is given;
// workgroup nblk + s computes shared expert s's gate logit  g = xn . f32(gate_w[s]) and stores
// sigmoid(g) = 1 / (1 + exp(-g)), the weight of that expert's output (engine.rs:6392-6425).
struct PrologueArgs {
  const void* x;
  int x_dt;
  const uint16_t* norm_w;  // [D] f16 or null (no norm: the gates read x as given)
  float eps;
  int D;
  float* xn;               // [D] f32 (when norm_w)
  int nblk;                // workgroups writing xn
  const uint16_t* gate_w;  // [ns][D] f16 or null
  int ns;
  float* shared_w;         // [ns]
};

__global__ __launch_bounds__(256) void k_moe_prologue(PrologueArgs a) {
  const int b = (int)blockIdx.x, tid = (int)threadIdx.x;
  const float inv = a.norm_w ? wg_inv_rms((const float*)a.x, a.D, a.eps) : 1.0f;
  auto xn_at = [&](int d) {
    return a.norm_w ? norm_elem(((const float*)a.x)[d], inv, a.norm_w[d])
                    : load_act(a.x, a.x_dt, (size_t)d);
  };
  if (b < a.nblk) {
    const int d0 = b * 1024;
    for (int d = d0 + tid; d < min(a.D, d0 + 1024); d += 256) a.xn[d] = xn_at(d);
    return;
  }
  const int s = b - a.nblk;
  const uint16_t* gw = a.gate_w + (size_t)s * a.D;
  float acc = 0.0f;
  for (int d = tid; d < a.D; d += 256) acc = __builtin_fmaf(xn_at(d), f16_to_f32(gw[d]), acc);
  __shared__ float red[4];
  acc = wave_sum(acc);
  if ((tid & 63) == 0) red[tid >> 6] = acc;
  __syncthreads();
  if (tid == 0) {
    const float g = (red[0] + red[1]) + (red[2] + red[3]);
    a.shared_w[s] = 1.0f / (1.0f + expf(-g));
  }
}

int launch_moe_prologue(const void* x, int x_dt, const uint16_t* norm_w, float eps, int D,
                        float* xn, const uint16_t* gate_w, int ns, float* shared_w,
                        hipStream_t st) {
  PrologueArgs a{x, x_dt, norm_w, eps, D, xn, norm_w ? (D + 1023) / 1024 : 0, gate_w,
                 gate_w ? ns : 0, shared_w};
  const int grid = a.nblk + a.ns;
  if (grid == 0) return 0;
  hipLaunchKernelGGL(k_moe_prologue, dim3((unsigned)grid), dim3(256), 0, st, a);
  VIB3_RETURN_LAUNCH();
}

}  // namespace vib3

using namespace vib3;

extern "C" {

int vib3_launch_rms_norm_f32(const void* input, void* output, const void* weight, int hidden_dim,
                             float eps, void* stream) {
  if (hidden_dim <= 0) return VIB3_ERR_BAD_COUNT;
  if (!input || !output || !weight) return VIB3_ERR_BAD_POINTER;
  hipLaunchKernelGGL(k_rms_norm<false>, dim3((unsigned)((hidden_dim + 1023) / 1024)), dim3(256),
                     0, (hipStream_t)stream, (const float*)input, output,
                     (const uint16_t*)weight, hidden_dim, eps);
  VIB3_RETURN_LAUNCH();
}

int vib3_launch_rms_norm_f32_to_f16(const void* input, void* output, const void* weight,
                                    int hidden_dim, float eps, void* stream) {
  if (hidden_dim <= 0) return VIB3_ERR_BAD_COUNT;
  if (!input || !output || !weight) return VIB3_ERR_BAD_POINTER;
  hipLaunchKernelGGL(k_rms_norm<true>, dim3((unsigned)((hidden_dim + 1023) / 1024)), dim3(256),
                     0, (hipStream_t)stream, (const float*)input, output,
                     (const uint16_t*)weight, hidden_dim, eps);
  VIB3_RETURN_LAUNCH();
}

int vib3_launch_residual_add_f32_f32(void* accumulator, const void* layer_output, int dim,
                                     void* stream) {
  if (dim < 0) return VIB3_ERR_BAD_COUNT;
  if (dim == 0) return 0;
  if (!accumulator || !layer_output) return VIB3_ERR_BAD_POINTER;
  hipLaunchKernelGGL(k_residual_add, dim3((unsigned)((dim + 255) / 256)), dim3(256), 0,
                     (hipStream_t)stream, (float*)accumulator, (const float*)layer_output, dim);
  VIB3_RETURN_LAUNCH();
}

int vib3_launch_sigmoid_gated_accumulate_f32(void* output, const void* expert_output,
                                             const void* gate_dev, int dim, void* stream) {
  if (dim < 0) return VIB3_ERR_BAD_COUNT;
  if (dim == 0) return 0;
  if (!output || !expert_output || !gate_dev) return VIB3_ERR_BAD_POINTER;
  hipLaunchKernelGGL(k_sigmoid_gated_acc, dim3((unsigned)((dim + 255) / 256)), dim3(256), 0,
                     (hipStream_t)stream, (float*)output, (const uint16_t*)expert_output,
                     (const float*)gate_dev, dim);
  VIB3_RETURN_LAUNCH();
}

}  // extern "C"
