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
#include "norm.h"

namespace vib3 {

// Inverse RMS of x[0..D) for a 256-thread workgroup, in the reference's summation order.
// Up to 8192 elements every load is issued before the first add (one round trip).
__device__ float wg_inv_rms(const float* x, int D, float eps) {
  const int tid = (int)threadIdx.x;
  float p = 0.0f;
  if (D <= 256 * 32) {
    float v[32];
#pragma unroll
    for (int i = 0; i < 32; i++) v[i] = tid + 256 * i < D ? x[tid + 256 * i] : 0.0f;
#pragma unroll
    for (int i = 0; i < 32; i++) p = __builtin_fmaf(v[i], v[i], p);
  } else {
    for (int d = tid; d < D; d += 256) {
      const float v = x[d];
      p = __builtin_fmaf(v, v, p);
    }
  }
  return block_inv_rms(p, D, eps);
}

__device__ __forceinline__ float norm_elem(float x, float inv, uint16_t w) {
  return norm_mul(x, inv, f16_to_f32(w));
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
// Thread t holds elements t + 256 i (i < kProMax, D <= 256 * kProMax): the layout of the
// reference's partial sums, so every load of a workgroup is issued at once (one round trip)
// and the normalised values it writes are already in its registers.
constexpr int kProMax = kNormMax;

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

template <int XDT>
__global__ __launch_bounds__(256) void k_moe_prologue(PrologueArgs a) {
  const int b = (int)blockIdx.x, tid = (int)threadIdx.x;
  const bool gate = b >= a.nblk;
  const int D = a.D;
  float xv[kProMax], wv[kProMax], gv[kProMax];
  // raw loads first, all unconditional (indices past D clamp to 0 and are zeroed after), so
  // the whole workgroup's data is one round trip
  uint32_t xr[kProMax];
  uint16_t wr[kProMax], gr[kProMax];
  const uint16_t* nw = a.norm_w ? a.norm_w : (const uint16_t*)a.x;
  const uint16_t* gw = gate ? a.gate_w + (size_t)(b - a.nblk) * D : (const uint16_t*)a.x;
#pragma unroll
  for (int i = 0; i < kProMax; i++) {
    const int d = tid + 256 * i < D ? tid + 256 * i : 0;
    xr[i] = XDT == VIB3_DT_F32 ? ((const uint32_t*)a.x)[d] : ((const uint16_t*)a.x)[d];
    wr[i] = nw[d];
    gr[i] = gw[d];
  }
#pragma unroll
  for (int i = 0; i < kProMax; i++) {
    const bool in = tid + 256 * i < D;
    const float xf = XDT == VIB3_DT_F32   ? __uint_as_float(xr[i])
                     : XDT == VIB3_DT_F16 ? f16_to_f32((uint16_t)xr[i])
                                          : bf16_to_f32((uint16_t)xr[i]);
    xv[i] = in ? xf : 0.0f;
    wv[i] = a.norm_w ? f16_to_f32(wr[i]) : 1.0f;
    gv[i] = in && gate ? f16_to_f32(gr[i]) : 0.0f;
  }
  float inv = 1.0f;
  if (a.norm_w) {
    float p = 0.0f;
#pragma unroll
    for (int i = 0; i < kProMax; i++) p = __builtin_fmaf(xv[i], xv[i], p);  // zeros past D
    inv = block_inv_rms(p, D, a.eps);
#pragma unroll
    for (int i = 0; i < kProMax; i++) xv[i] = norm_mul(xv[i], inv, wv[i]);
  }
  if (!gate) {
    // this workgroup's 1024 elements: i = 4b .. 4b + 3
#pragma unroll
    for (int i = 0; i < kProMax; i++) {
      const int d = tid + 256 * i;
      if (i / 4 == b && d < D) a.xn[d] = xv[i];
    }
    return;
  }
  float acc = 0.0f;
#pragma unroll
  for (int i = 0; i < kProMax; i++) acc = __builtin_fmaf(xv[i], gv[i], acc);
  __shared__ float red[4];
  acc = wave_sum(acc);
  if ((tid & 63) == 0) red[tid >> 6] = acc;
  __syncthreads();
  if (tid == 0) {
    const float g = (red[0] + red[1]) + (red[2] + red[3]);
    a.shared_w[b - a.nblk] = 1.0f / (1.0f + expf(-g));
  }
}

int launch_moe_prologue(const void* x, int x_dt, const uint16_t* norm_w, float eps, int D,
                        float* xn, const uint16_t* gate_w, int ns, float* shared_w,
                        hipStream_t st) {
  if (D > 256 * kProMax) return VIB3_ERR_UNSUPPORTED;
  PrologueArgs a{x, x_dt, norm_w, eps, D, xn, norm_w ? (D + 1023) / 1024 : 0, gate_w,
                 gate_w ? ns : 0, shared_w};
  const int grid = a.nblk + a.ns;
  if (grid == 0) return 0;
  if (x_dt == VIB3_DT_F32)
    hipLaunchKernelGGL(k_moe_prologue<VIB3_DT_F32>, dim3((unsigned)grid), dim3(256), 0, st, a);
  else if (x_dt == VIB3_DT_F16)
    hipLaunchKernelGGL(k_moe_prologue<VIB3_DT_F16>, dim3((unsigned)grid), dim3(256), 0, st, a);
  else
    hipLaunchKernelGGL(k_moe_prologue<VIB3_DT_BF16>, dim3((unsigned)grid), dim3(256), 0, st, a);
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
