// api.hip — the C ABI of libvib3_hip (include/vib3_hip.h): argument checks, workspace layout
// and launch sequences. All entry points are asynchronous on the caller's stream and allocate
// nothing. They keep no mutable global state, so they are reentrant across streams, except
// vib3_launch_moe_int4_layer_noalloc, whose calls share one device scratch per GPU.
#include <string.h>

#include <atomic>

#include "common.h"
#include "kernels.h"

using namespace vib3;

namespace {

inline hipStream_t S(void* p) { return (hipStream_t)p; }
inline bool aligned16(const void* p) { return ((uintptr_t)p & 15) == 0; }
inline bool valid_act_dt(int dt) { return dt == VIB3_DT_F32 || dt == VIB3_DT_F16 || dt == VIB3_DT_BF16; }
inline bool valid_scale_dt(int dt) { return dt == VIB3_DT_F16 || dt == VIB3_DT_BF16; }
inline bool valid_out_dt(int dt) { return dt == VIB3_DT_F32 || dt == VIB3_DT_F16; }
inline size_t round_up(size_t v, size_t a) { return (v + a - 1) / a * a; }

// One flat INT4 matrix (or up/gate pair) times a vector: the fast kernel when the shape and
// alignment allow 16-byte chunk loads, otherwise the generic kernel.
int int4_flat(const void* x, int x_dt, const void* d0, const void* s0, const void* d1,
              const void* s1, void* out, int out_dt, int k, int m, int g, int sdt, bool dual,
              hipStream_t st) {
  if (k <= 0 || m < 0 || g <= 0) return VIB3_ERR_BAD_COUNT;
  if (!x || !d0 || !s0 || !out || (dual && (!d1 || !s1))) return VIB3_ERR_BAD_POINTER;
  if (m == 0) return 0;
  const bool fast = (k % 32 == 0) && (k / 32 <= 16 * kWave) && aligned16(d0) &&
                    (!dual || aligned16(d1)) && aligned16(x) && ((uintptr_t)s0 % 2 == 0) &&
                    (!dual || (uintptr_t)s1 % 2 == 0);
  if (fast) {
    RowsArgs a{};
    a.x = x; a.x_dt = x_dt; a.K = k; a.M = m; a.g = g; a.sdt = sdt; a.nslots = 1;
    a.flat0 = MatRef{nullptr, (const uint8_t*)d0, (const uint16_t*)s0, 0, m, 0};
    a.flat1 = dual ? MatRef{nullptr, (const uint8_t*)d1, (const uint16_t*)s1, 0, m, 0} : a.flat0;
    a.out = out; a.out_dt = out_dt; a.out_stride = 0;
    return launch_rows(a, dual, st);
  }
  GenericArgs a{x, x_dt, k, m, g, sdt, (const uint8_t*)d0, (const uint16_t*)s0,
                (const uint8_t*)d1, (const uint16_t*)s1, out, out_dt};
  return launch_generic(a, dual, st);
}

inline const void* scales_of(const void* page, int k, int m) {
  return (const uint8_t*)page + (size_t)((k + 1) / 2) * (size_t)m;
}

__global__ void k_silu_mul(const uint16_t* a, const uint16_t* b, uint16_t* out, int n) {
  const int i = (int)(blockIdx.x * blockDim.x + threadIdx.x);
  if (i >= n) return;
  const float g = f16_to_f32(a[i]);
  out[i] = f32_to_f16_bits((g / (1.0f + expf(-g))) * f16_to_f32(b[i]));
}

__global__ void k_weighted_acc(float* out, const void* e, int e_f32, float w, int n) {
  const int i = (int)(blockIdx.x * blockDim.x + threadIdx.x);
  if (i >= n) return;
  const float v = e_f32 ? ((const float*)e)[i] : f16_to_f32(((const uint16_t*)e)[i]);
  out[i] = add_mul_rn(out[i], w, v);
}

__global__ void k_weighted_acc_f16(uint16_t* out, const uint16_t* e, const float* wdev, float w,
                                   int n) {
  const int i = (int)(blockIdx.x * blockDim.x + threadIdx.x);
  if (i >= n) return;
  if (wdev) w = wdev[0];
  out[i] = f32_to_f16_bits(add_mul_rn(f16_to_f32(out[i]), w, f16_to_f32(e[i])));
}

__global__ void k_weighted_acc_dev(float* out, const uint16_t* e, const float* wdev, int n) {
  const int i = (int)(blockIdx.x * blockDim.x + threadIdx.x);
  if (i >= n) return;
  out[i] = add_mul_rn(out[i], wdev[0], f16_to_f32(e[i]));
}

__global__ void k_zero(uint4* p16, size_t n16, uint8_t* tail, size_t ntail) {
  const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n16) p16[i] = make_uint4(0, 0, 0, 0);
  if (i < ntail) tail[i] = 0;
}

// Workspace of the fused layer: [scores[E] | ids[k] | wts[k] | router slots u64[E] |
// status: error i32, router tag u32 | h[nslots][inter] | xn f32[hidden] (with a norm) |
// shared weights f32[num_shared] (gated) | down page addresses u64[nslots][down pages]].
struct LayerWs {
  size_t scores, ids, wts, slots, error, h, xn, shared_w, dbase, total;
  int down_pages;  // pages of one down matrix (whole layer launches of a paged layer)
};

// The no-allocation entry point's device memory: the layer workspace of
// vib3_launch_moe_int4_layer_noalloc, at most kNoAllocScratchBytes. Every GPU the library runs
// on holds its own copy (zero when the code object loads, which is the state the router tags
// need) until the process ends. In host code `scratch` is only a symbol handle: its device
// address, per device, comes from hipGetSymbolAddress (noalloc_scratch).
constexpr size_t kNoAllocScratchBytes = 256 * 1024;
static __device__ __align__(256) uint8_t scratch[kNoAllocScratchBytes];

// Device address of this device's `scratch`, looked up once per device (set-up of the first
// call on that device), or null if the lookup failed.
char* noalloc_scratch() {
  static std::atomic<char*> ptrs[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return nullptr;
  char* p = ptrs[dev].load(std::memory_order_acquire);
  if (!p) {
    void* addr = nullptr;
    if (hipGetSymbolAddress(&addr, HIP_SYMBOL(scratch)) != hipSuccess || !addr) return nullptr;
    p = (char*)addr;
    ptrs[dev].store(p, std::memory_order_release);
  }
  return p;
}

// Routing mode of a layer call (see RowsArgs::route).
int router_mode(const vib3_moe_int4_layer* L) {
  if (!L->router_w || L->top_k <= 0) return kRouteGiven;
  int mode = L->num_experts <= kMaxExpertsInKernel ? 2 : 0;
#ifdef VIB3_ROUTE_MODE  // (profiling builds: 0 separate selection launch, 1 selection from
                        // the router kernel's scores in the gate/up prologue, 2 fused)
  mode = L->num_experts <= kMaxExpertsInKernel ? VIB3_ROUTE_MODE : 0;
#endif
  return mode == 2 ? kRouteFused : mode == 1 ? kRouteScores : kRouteGiven;
}

// Router tag of a stage-by-stage timing launch (vib3_launch_moe_int4_layer_stage): a
// process-wide counter with bit 31 set, so it never equals 0 (a zeroed slot) nor a device tag
// (next_tag keeps those below 2^31). Whole-layer launches take their tag on the device.
uint32_t stage_generation() {
  static std::atomic<uint32_t> gen{0};
  return 0x80000000u | (gen.fetch_add(1, std::memory_order_relaxed) & 0x7fffffffu);
}

// scratch = true: the layout of the no-allocation scratch, whose status words (error, tag)
// and router slots sit at fixed offsets for every layer shape: calls with different shapes
// reuse the same bytes, and a slot must only ever hold an older tag of the same tag word.
LayerWs layer_ws(const vib3_moe_int4_layer* L, bool scratch = false) {
  LayerWs w{};
  const int nslots = L->top_k + L->num_shared;
  const size_t hsz = (L->flags & VIB3_MOE_F32_INTERMEDIATE) ? 4 : 2;
  const size_t E = (size_t)(L->num_experts > 0 ? L->num_experts : 0);
  if (scratch) {
    w.error = 0;
    w.slots = 256;
    w.scores = round_up(w.slots + 8 * (size_t)kMaxExpertsInKernel, 256);
  } else {
    w.scores = 0;
  }
  w.ids = round_up(w.scores + 4 * E, 256);
  w.wts = round_up(w.ids + 2 * (size_t)(L->top_k > 0 ? L->top_k : 0), 256);
  size_t next = round_up(w.wts + 4 * (size_t)(L->top_k > 0 ? L->top_k : 0), 256);
  if (!scratch) {
    w.slots = next;
    w.error = round_up(w.slots + 8 * E, 256);
    next = round_up(w.error + 8, 256);  // error word, then the router tag word at error + 4
  }
  w.h = next;
  w.xn = round_up(w.h + hsz * (size_t)(nslots > 0 ? nslots : 0) * (size_t)(L->inter > 0 ? L->inter : 0), 256);
  w.shared_w = round_up(w.xn + (L->norm_weight ? 4 * (size_t)(L->hidden > 0 ? L->hidden : 0) : 0), 256);
  w.dbase = round_up(w.shared_w + (L->shared_gate ? 4 * (size_t)(L->num_shared > 0 ? L->num_shared : 0) : 0), 256);
  const int rpp = L->rows_per_page[2];
  w.down_pages = rpp > 0 && L->hidden > 0 ? (L->hidden + rpp - 1) / rpp : 0;
  w.total = round_up(w.dbase + 8 * (size_t)(nslots > 0 ? nslots : 0) * (size_t)w.down_pages, 256);
  return w;
}

}  // namespace

#ifndef VIB3_DOWN_LIST
#define VIB3_DOWN_LIST 1  // (build-time switch: the gate/up kernel lists the down pages)
#endif

extern "C" {

const char* vib3_hip_version(void) { return "vib3_hip 0.1 gfx950"; }

int vib3_hip_zero(void* ptr, size_t bytes, void* stream) {
  if (!ptr) return VIB3_ERR_BAD_POINTER;
  if (bytes == 0) return 0;
  size_t n16 = aligned16(ptr) ? bytes / 16 : 0;
  uint8_t* tail = (uint8_t*)ptr + n16 * 16;
  size_t ntail = bytes - n16 * 16;
  size_t n = n16 > ntail ? n16 : ntail;
  hipLaunchKernelGGL(k_zero, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, S(stream),
                     (uint4*)ptr, n16, tail, ntail);
  VIB3_RETURN_LAUNCH();
}

// ---------------------------------------------------------------- reference-compatible

int vib3_launch_partial_matmul_int4(const void* input, const void* weight_packed,
                                    const void* scales, void* output, int k, int m_slice,
                                    int group_size, void* stream) {
  return int4_flat(input, VIB3_DT_F16, weight_packed, scales, nullptr, nullptr, output,
                   VIB3_DT_F16, k, m_slice, group_size, VIB3_DT_F16, false, S(stream));
}

int vib3_launch_partial_matmul_int4_f32(const void* input, const void* weight, const void* scales,
                                        void* output, int k, int m_slice, int group_size,
                                        void* stream) {
  return int4_flat(input, VIB3_DT_F32, weight, scales, nullptr, nullptr, output, VIB3_DT_F16, k,
                   m_slice, group_size, VIB3_DT_F16, false, S(stream));
}

int vib3_launch_fused_swiglu_int4_f32(const void* input, const void* up_weight,
                                      const void* up_scales, const void* gate_weight,
                                      const void* gate_scales, void* output, int k, int m_slice,
                                      int group_size, void* stream) {
  return int4_flat(input, VIB3_DT_F32, up_weight, up_scales, gate_weight, gate_scales, output,
                   VIB3_DT_F16, k, m_slice, group_size, VIB3_DT_F16, true, S(stream));
}

int vib3_launch_silu_mul(const void* up_result, const void* gate_result, void* output, int dim,
                         void* stream) {
  if (dim < 0) return VIB3_ERR_BAD_COUNT;
  if (!up_result || !gate_result || !output) return VIB3_ERR_BAD_POINTER;
  if (dim == 0) return 0;
  hipLaunchKernelGGL(k_silu_mul, dim3((unsigned)((dim + 255) / 256)), dim3(256), 0, S(stream),
                     (const uint16_t*)up_result, (const uint16_t*)gate_result, (uint16_t*)output,
                     dim);
  VIB3_RETURN_LAUNCH();
}

int vib3_launch_weighted_accumulate_f32(void* output, const void* expert_output, float weight,
                                        int dim, void* stream) {
  if (dim < 0) return VIB3_ERR_BAD_COUNT;
  if (!output || !expert_output) return VIB3_ERR_BAD_POINTER;
  if (dim == 0) return 0;
  hipLaunchKernelGGL(k_weighted_acc, dim3((unsigned)((dim + 255) / 256)), dim3(256), 0,
                     S(stream), (float*)output, expert_output, 0, weight, dim);
  VIB3_RETURN_LAUNCH();
}

int vib3_launch_weighted_accumulate(void* output, const void* expert_output, float weight,
                                    int dim, void* stream) {
  if (dim < 0) return VIB3_ERR_BAD_COUNT;
  if (!output || !expert_output) return VIB3_ERR_BAD_POINTER;
  if (dim == 0) return 0;
  hipLaunchKernelGGL(k_weighted_acc_f16, dim3((unsigned)((dim + 255) / 256)), dim3(256), 0,
                     S(stream), (uint16_t*)output, (const uint16_t*)expert_output, nullptr,
                     weight, dim);
  VIB3_RETURN_LAUNCH();
}

int vib3_launch_weighted_accumulate_f32_dev_scalar(void* output, const void* expert_output,
                                                   const void* dev_weight, int dim,
                                                   void* stream) {
  if (dim < 0) return VIB3_ERR_BAD_COUNT;
  if (!output || !expert_output || !dev_weight) return VIB3_ERR_BAD_POINTER;
  if (dim == 0) return 0;
  hipLaunchKernelGGL(k_weighted_acc_dev, dim3((unsigned)((dim + 255) / 256)), dim3(256), 0,
                     S(stream), (float*)output, (const uint16_t*)expert_output,
                     (const float*)dev_weight, dim);
  VIB3_RETURN_LAUNCH();
}

int vib3_launch_weighted_accumulate_f32_f32(void* output, const void* expert_output,
                                            float weight, int dim, void* stream) {
  if (dim < 0) return VIB3_ERR_BAD_COUNT;
  if (!output || !expert_output) return VIB3_ERR_BAD_POINTER;
  if (dim == 0) return 0;
  hipLaunchKernelGGL(k_weighted_acc, dim3((unsigned)((dim + 255) / 256)), dim3(256), 0,
                     S(stream), (float*)output, expert_output, 1, weight, dim);
  VIB3_RETURN_LAUNCH();
}

int vib3_launch_router_gemv(const void* hidden_state, const void* router_weights, float* scores,
                            int hidden_dim, int num_experts, void* stream) {
  if (hidden_dim <= 0 || num_experts <= 0) return VIB3_ERR_BAD_COUNT;
  if (!hidden_state || !router_weights || !scores) return VIB3_ERR_BAD_POINTER;
  RouterArgs a{};
  a.x = hidden_state; a.x_dt = VIB3_DT_F16; a.w = router_weights; a.w_dt = VIB3_DT_F16;
  a.D = hidden_dim; a.E = num_experts; a.scores = scores;
  return launch_router_logits(a, S(stream));
}

int vib3_launch_router_gemv_f32(const void* hidden_state, const void* router_weights,
                                float* scores, int hidden_dim, int num_experts, void* stream) {
  if (hidden_dim <= 0 || num_experts <= 0) return VIB3_ERR_BAD_COUNT;
  if (!hidden_state || !router_weights || !scores) return VIB3_ERR_BAD_POINTER;
  RouterArgs a{};
  a.x = hidden_state; a.x_dt = VIB3_DT_F32; a.w = router_weights; a.w_dt = VIB3_DT_F16;
  a.D = hidden_dim; a.E = num_experts; a.scores = scores;
  return launch_router_logits(a, S(stream));
}

int vib3_launch_router_topk(const void* hidden_state, const void* router_weights,
                            float* scores_buf, const float* bias, uint16_t* out_ids,
                            float* out_weights, int hidden_dim, int num_experts, int top_k,
                            int scoring_mode, float scaling_factor, void* stream) {
  if (hidden_dim <= 0 || num_experts <= 0 || num_experts > kMaxExperts || top_k <= 0 ||
      top_k > num_experts || top_k > 64)
    return VIB3_ERR_BAD_COUNT;
  if (scoring_mode != VIB3_ROUTER_SOFTMAX && scoring_mode != VIB3_ROUTER_SIGMOID)
    return VIB3_ERR_UNSUPPORTED;
  if (!hidden_state || !router_weights || !scores_buf || !out_ids || !out_weights)
    return VIB3_ERR_BAD_POINTER;
  RouterArgs a{};
  a.x = hidden_state; a.x_dt = VIB3_DT_F32; a.w = router_weights; a.w_dt = VIB3_DT_F16;
  a.bias = bias; a.D = hidden_dim; a.E = num_experts; a.top_k = top_k; a.mode = scoring_mode;
  a.scaling = scoring_mode == VIB3_ROUTER_SIGMOID ? scaling_factor : 1.0f;
  a.normalize = 1;  // the reference GPU kernel always normalises (kernels.cu:4056)
  a.scores = scores_buf; a.ids = out_ids; a.wts = out_weights;
  int rc = launch_router_logits(a, S(stream));
  if (rc) return rc;
  return launch_router_select(a, S(stream));
}

// ---------------------------------------------------------------- additive

int vib3_launch_partial_matmul_int4_ex(const void* input, int input_dtype, const void* weight_page,
                                       void* output, int output_dtype, int k, int m_slice,
                                       int group_size, int scale_dtype, void* stream) {
  if (!valid_act_dt(input_dtype) || !valid_out_dt(output_dtype) || !valid_scale_dt(scale_dtype))
    return VIB3_ERR_UNSUPPORTED;
  if (k <= 0 || m_slice < 0) return VIB3_ERR_BAD_COUNT;
  return int4_flat(input, input_dtype, weight_page, scales_of(weight_page, k, m_slice), nullptr,
                   nullptr, output, output_dtype, k, m_slice, group_size, scale_dtype, false,
                   S(stream));
}

int vib3_launch_partial_swiglu_int4_ex(const void* input, int input_dtype, const void* up_page,
                                       const void* gate_page, void* output, int output_dtype,
                                       int k, int m_slice, int group_size, int scale_dtype,
                                       void* stream) {
  if (!valid_act_dt(input_dtype) || !valid_out_dt(output_dtype) || !valid_scale_dt(scale_dtype))
    return VIB3_ERR_UNSUPPORTED;
  if (k <= 0 || m_slice < 0) return VIB3_ERR_BAD_COUNT;
  return int4_flat(input, input_dtype, up_page, scales_of(up_page, k, m_slice), gate_page,
                   scales_of(gate_page, k, m_slice), output, output_dtype, k, m_slice, group_size,
                   scale_dtype, true, S(stream));
}

size_t vib3_router_workspace_bytes(int num_experts) {
  return round_up(4 * (size_t)(num_experts > 0 ? num_experts : 0), 256) + 256 + 256;
}

int vib3_launch_router_topk_ex(const void* hidden, int hidden_dtype, const void* router_weights,
                               int weight_dtype, const float* bias, int hidden_dim,
                               int num_experts, int top_k, int scoring_mode, float scaling_factor,
                               int normalize, float* scores_out, uint16_t* out_ids,
                               float* out_weights, void* workspace, void* stream) {
  if (!valid_act_dt(hidden_dtype) || !valid_act_dt(weight_dtype)) return VIB3_ERR_UNSUPPORTED;
  if (scoring_mode != VIB3_ROUTER_SOFTMAX && scoring_mode != VIB3_ROUTER_SIGMOID)
    return VIB3_ERR_UNSUPPORTED;
  if (hidden_dim <= 0 || num_experts <= 0 || num_experts > kMaxExperts || top_k <= 0 ||
      top_k > num_experts || top_k > 64)
    return VIB3_ERR_BAD_COUNT;
  if (!hidden || !router_weights || !workspace) return VIB3_ERR_BAD_POINTER;
  char* ws = (char*)workspace;
  const size_t sc = 0, ids = round_up(4 * (size_t)num_experts, 256), wts = ids + 256;
  RouterArgs a{};
  a.x = hidden; a.x_dt = hidden_dtype; a.w = router_weights; a.w_dt = weight_dtype;
  a.bias = bias; a.D = hidden_dim; a.E = num_experts; a.top_k = top_k; a.mode = scoring_mode;
  a.scaling = scoring_mode == VIB3_ROUTER_SIGMOID ? scaling_factor : 1.0f;
  a.normalize = normalize;
  a.scores = scores_out ? scores_out : (float*)(ws + sc);
  a.ids = (uint16_t*)(ws + ids);
  a.wts = (float*)(ws + wts);
  a.out_ids = out_ids;
  a.out_wts = out_weights;
  const int rc = launch_router_logits(a, S(stream));
  if (rc) return rc;
  return launch_router_select(a, S(stream));
}

size_t vib3_moe_int4_workspace_bytes(const vib3_moe_int4_layer* L) {
  if (!L) return 0;
  return layer_ws(L).total;
}

// only < 0: the whole layer; only = 0 / 1 / 2: just the router / gate-up / down launches, which
// read what the earlier stages of a previous call left in the workspace (stage timing).
// scratch: the no-allocation entry point's device scratch (used instead of L->workspace,
// in its fixed layout), or null.
static int moe_int4_layer(const vib3_moe_int4_layer* L, void* stream, int only,
                          char* scratch = nullptr) {
  if (!L) return VIB3_ERR_BAD_POINTER;
  if (!valid_act_dt(L->x_dtype) || !valid_scale_dt(L->scale_dtype)) return VIB3_ERR_UNSUPPORTED;
  if (L->hidden <= 0 || L->inter <= 0 || L->group_size <= 0 || L->top_k < 0 ||
      L->num_shared < 0 || L->max_pages <= 0)
    return VIB3_ERR_BAD_COUNT;
  const int nslots = L->top_k + L->num_shared;
  if (nslots <= 0 || nslots > 16 || L->top_k > 64) return VIB3_ERR_BAD_COUNT;
  if (L->hidden % 32 || L->inter % 32) return VIB3_ERR_UNSUPPORTED;
  if (L->hidden >= 65536 || L->inter >= 65536) return VIB3_ERR_UNSUPPORTED;  // page_magic range
  for (int s = 0; s < 3; s++)
    if (L->rows_per_page[s] <= 0) return VIB3_ERR_BAD_COUNT;
  if ((L->rows_per_page[0] + 0LL) * L->max_pages < L->inter ||
      (L->rows_per_page[1] + 0LL) * L->max_pages < L->inter ||
      (L->rows_per_page[2] + 0LL) * L->max_pages < L->hidden)
    return VIB3_ERR_BAD_COUNT;
  if (!L->x || !L->out || (!scratch && (!L->workspace || !aligned16(L->workspace))) ||
      (L->top_k > 0 && !L->page_table) || (L->num_shared > 0 && !L->shared_page_table) ||
      !aligned16(L->x))
    return VIB3_ERR_BAD_POINTER;
  if (L->norm_weight && L->x_dtype != VIB3_DT_F32) return VIB3_ERR_UNSUPPORTED;  // f32 stream
  if ((L->norm_weight || L->shared_gate) && L->hidden > 8192) return VIB3_ERR_UNSUPPORTED;
  if (L->shared_gate && L->num_shared <= 0) return VIB3_ERR_BAD_COUNT;
  const LayerWs w = layer_ws(L, scratch != nullptr);
  if (w.total > (scratch ? kNoAllocScratchBytes : L->workspace_bytes)) return VIB3_ERR_WORKSPACE;
  char* ws = scratch ? scratch : (char*)L->workspace;
  hipStream_t st = S(stream);
  auto run = [&](int i) { return only < 0 || only == i; };

  // The activation the router and experts read: x, or RMSNorm(x). The gate/up kernel
  // normalises x itself and computes the shared experts' gates where it can (fused routing,
  // f32 stream in int16 chunks, hidden <= 8192); else the prologue kernel writes RMSNorm(x)
  // and the gates first (stage 0 with the router).
#ifndef VIB3_F32_SPLIT
#define VIB3_F32_SPLIT 0  // (profiling builds: f32 stream as hi + lo f16 pairs)
#endif
  const int x_i16 = VIB3_F32_SPLIT ? 0 : 1;  // f32 stream: int16 chunks
  bool fuse_prologue = false;
  if (L->norm_weight && !(L->flags & VIB3_MOE_SEPARATE_PROLOGUE)) {
    RowsArgs p{};
    p.x = L->x; p.x_dt = L->x_dtype; p.x_i16 = x_i16; p.K = L->hidden; p.M = L->inter;
    p.nslots = nslots; p.routed_table = L->page_table; p.route = router_mode(L);
    p.router.D = L->hidden; p.router.w = L->router_w; p.router.x = L->x;
    p.router.E = L->num_experts;
    p.norm_w = (const uint16_t*)L->norm_weight;
    p.gate_w = (const uint16_t*)L->shared_gate;
    p.ngate = L->shared_gate ? L->num_shared : 0;
    fuse_prologue = rows_fuse_prologue(p);
  }
  const void* xa = L->norm_weight && !fuse_prologue ? (const void*)(ws + w.xn) : L->x;
  const float* shared_w = L->shared_gate ? (const float*)(ws + w.shared_w) : nullptr;
  if (run(0) && !fuse_prologue && (L->norm_weight || L->shared_gate)) {
    const int rc = launch_moe_prologue(L->x, L->x_dtype, (const uint16_t*)L->norm_weight,
                                       L->norm_eps, L->hidden, (float*)(ws + w.xn),
                                       (const uint16_t*)L->shared_gate, L->num_shared,
                                       (float*)(ws + w.shared_w), st);
    if (rc) return rc;
  }

  const uint16_t* ids = (const uint16_t*)(ws + w.ids);
  const float* wts = (const float*)(ws + w.wts);
  RouterArgs router{};
  int route = kRouteGiven;
  if (L->top_k > 0) {
    if (L->router_w) {
      if (!valid_act_dt(L->router_w_dtype)) return VIB3_ERR_UNSUPPORTED;
      if (L->num_experts <= 0 || L->num_experts > kMaxExperts || L->top_k > L->num_experts)
        return VIB3_ERR_BAD_COUNT;
      if (L->scoring_mode != VIB3_ROUTER_SOFTMAX && L->scoring_mode != VIB3_ROUTER_SIGMOID)
        return VIB3_ERR_UNSUPPORTED;
      router.x = xa; router.x_dt = L->x_dtype; router.w = L->router_w;
      router.w_dt = L->router_w_dtype; router.bias = L->router_bias; router.D = L->hidden;
      router.E = L->num_experts; router.top_k = L->top_k; router.mode = L->scoring_mode;
      router.scaling = L->scoring_mode == VIB3_ROUTER_SIGMOID ? L->scaling_factor : 1.0f;
      router.normalize = L->normalize;
      router.scores = L->out_scores ? L->out_scores : (float*)(ws + w.scores);
      router.ids = (uint16_t*)(ws + w.ids);
      router.wts = (float*)(ws + w.wts);
      router.out_ids = L->out_ids;
      router.out_wts = L->out_weights;
      // up to 512 experts: logits and selection inside the gate/up kernel (fused); larger
      // counts: the router kernel plus a selection launch. VIB3_ROUTE_MODE (tuning/diagnosis)
      // forces 0 = separate selection launch, 1 = selection in the gate/up prologue from the
      // router kernel's scores, 2 = fused.
      route = router_mode(L);
      router.slots = (uint64_t*)(ws + w.slots);
      router.error = (int*)(ws + w.error);
      router.spin_limit = kRouterSpinLimit;
      if (L->flags & VIB3_MOE_TEST_ROUTER_TIMEOUT) {  // no slot matches: the wait gives up
        router.poll_xor = 0x40000000u;
        router.spin_limit = 64;
      }
      // whole layer: the tag lives in the workspace and advances on the device (graph
      // replays get a new tag each); one stage alone: a host tag (the down kernel that would
      // advance the word may not run)
      if (only < 0 && route == kRouteFused) router.gen_word = (uint32_t*)(ws + w.error + 4);
      else router.gen = stage_generation();
      if (run(0) && route != kRouteFused) {
        int rc = launch_router_logits(router, st);
        if (rc) return rc;
        if (route == kRouteGiven) {  // selection kernel publishes ids / weights
          rc = launch_router_select(router, st);
          if (rc) return rc;
        }
      }
    } else {
      if (!L->in_ids || !L->in_weights) return VIB3_ERR_BAD_POINTER;
      ids = L->in_ids;
      wts = L->in_weights;
    }
  }

  const int h_dt = (L->flags & VIB3_MOE_F32_INTERMEDIATE) ? VIB3_DT_F32 : VIB3_DT_F16;
  RowsArgs a{};
  a.x = xa; a.x_dt = L->x_dtype; a.K = L->hidden; a.M = L->inter; a.g = L->group_size;
  a.sdt = L->scale_dtype; a.nslots = nslots;
  a.routed_table = L->page_table; a.shared_table = L->shared_page_table; a.ids = ids;
  a.top_k = L->top_k; a.max_pages = L->max_pages;
  for (int q = 0; q < 3; q++) {
    a.rpp[q] = L->rows_per_page[q];
    a.magic[q] = page_magic(L->rows_per_page[q]);
  }
  a.out = ws + w.h; a.out_dt = h_dt; a.out_stride = (size_t)L->inter;
  a.route = route;
  a.router = router;
  a.x_i16 = x_i16;
#ifndef VIB3_PRE_SHARED
#define VIB3_PRE_SHARED 1  // (profiling builds: 0 = no shared items before the selection)
#endif
  a.pre_shared = VIB3_PRE_SHARED;
  if (fuse_prologue) {
    a.norm_w = (const uint16_t*)L->norm_weight;
    a.eps = L->norm_eps;
    a.gate_w = (const uint16_t*)L->shared_gate;
    a.ngate = L->shared_gate ? L->num_shared : 0;
    a.shared_w = (float*)(ws + w.shared_w);
  }
  // the gate/up kernel lists the down page addresses for the down kernel (a down stage alone
  // reads the list its gate/up stage left, like h and the ids)
  const bool bases = VIB3_DOWN_LIST && w.down_pages > 0 && w.down_pages <= L->max_pages &&
                     rows_write_bases(a);
  if (bases) {
    a.down_bases = (uint64_t*)(ws + w.dbase);
    a.down_pages = w.down_pages;
  }
  if (run(1)) {
    int rc = launch_rows(a, true, st);
    if (rc) return rc;
  }

  DownArgs d{};
  d.h = ws + w.h; d.h_dt = h_dt; d.K = L->inter; d.M = L->hidden; d.g = L->group_size;
  d.sdt = L->scale_dtype; d.nslots = nslots; d.routed_table = L->page_table;
  d.shared_table = L->shared_page_table; d.ids = ids; d.wts = wts; d.top_k = L->top_k;
  d.max_pages = L->max_pages; d.rpp = L->rows_per_page[2];
  d.magic = page_magic(L->rows_per_page[2]);
  if (bases) {
    d.bases = (const uint64_t*)(ws + w.dbase);
    d.bases_stride = w.down_pages;
  }
  d.round_f16 = (L->flags & VIB3_MOE_F32_INTERMEDIATE) ? 0 : 1;
  d.out = L->out;
  d.residual = L->residual;
  d.shared_w = shared_w;
  d.gen_word = router.gen_word;
  return run(2) ? launch_down(d, st) : 0;
}

int vib3_launch_moe_int4_layer(const vib3_moe_int4_layer* L, void* stream) {
  return moe_int4_layer(L, stream, -1);
}

int vib3_launch_moe_int4_layer_noalloc(const vib3_moe_int4_layer* L, void* stream) {
  char* ws = noalloc_scratch();
  if (!ws) return VIB3_ERR_BAD_POINTER;
  return moe_int4_layer(L, stream, -1, ws);
}

int vib3_moe_int4_layer_status(const vib3_moe_int4_layer* L, int clear, void* stream) {
  if (!L) return VIB3_ERR_BAD_POINTER;
  // workspace NULL: the status of vib3_launch_moe_int4_layer_noalloc calls on this device
  char* base = L->workspace ? (char*)L->workspace : noalloc_scratch();
  if (!base) return VIB3_ERR_BAD_POINTER;
  const LayerWs w = layer_ws(L, !L->workspace);
  if (L->workspace && L->workspace_bytes < w.total) return VIB3_ERR_WORKSPACE;
  int* dev = (int*)(base + w.error);
  int host = 0;
  hipError_t e = hipMemcpyAsync(&host, dev, sizeof(int), hipMemcpyDeviceToHost, S(stream));
  if (e == hipSuccess) e = hipStreamSynchronize(S(stream));
  if (e != hipSuccess) return (int)e;
  if (clear && host) {
    const int rc = vib3_hip_zero(dev, sizeof(int), stream);
    if (rc) return rc;
    e = hipStreamSynchronize(S(stream));
    if (e != hipSuccess) return (int)e;
  }
  return host ? 1 : 0;
}

int vib3_moe_int4_router_fused(const vib3_moe_int4_layer* L) {
  return L && router_mode(L) == kRouteFused ? 1 : 0;
}

int vib3_launch_moe_int4_layer_stage(const vib3_moe_int4_layer* L, int stage, void* stream) {
  if (stage < 0 || stage > 2) return VIB3_ERR_BAD_COUNT;
  return moe_int4_layer(L, stream, stage);
}

}  // extern "C"
