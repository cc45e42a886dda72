/*
 * vib3_hip.h — C ABI of the MI355X (gfx950) MoE expert compute library, libvib3_hip.so.
 *
 * Drop-in for the MoE/router part of vib3's `extern "C"` launcher interface
 * (threehundobaud/vic: src/compute/cuda_ffi.rs:143-1063, implemented there by
 * cuda/src/kernels.cu). Conventions kept from the reference:
 *   - every launcher is asynchronous on `stream` (a hipStream_t; NULL = the null stream);
 *   - the return value is 0 on success, a positive hipError_t on a HIP error, and negative for
 *     argument errors (-1 unsupported shape/dtype, -2 bad count, as kernels.cu:5671-5672;
 *     -3 bad pointer/alignment, -4 workspace too small);
 *   - all buffers are caller-owned device pointers; nothing here allocates device memory;
 *   - INT4 pages are laid out as [m x ceil(k/2)] packed nibbles (low nibble = even column,
 *     stored q = code + 8) followed by [m x ceil(k/g)] little-endian 2-byte scales
 *     (kernels.rs:95-98, :3752-3825); dequantised weight = (q - 8) * scale.
 *     A scale that is not finite or not > 0 decodes as 1/8, as the CPU fallback does
 *     (kernels.rs:2791-2797).
 *
 * Fast paths need k % 32 == 0 and 16-byte aligned rows (k/2 % 16 == 0, page bases 16-byte
 * aligned); other shapes run a simple HIP kernel with the same results. Activations given as
 * f32 or bf16 must satisfy |x| < 65504 (the reference CPU path holds them in f16).
 */
#ifndef VIB3_HIP_H
#define VIB3_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* element types */
#define VIB3_DT_F32 0
#define VIB3_DT_F16 1
#define VIB3_DT_BF16 2

/* router scoring modes (kernels.rs:2226 RouterScoringFunc) */
#define VIB3_ROUTER_SOFTMAX 0
#define VIB3_ROUTER_SIGMOID 1

/* error codes besides hipError_t */
#define VIB3_ERR_UNSUPPORTED (-1)
#define VIB3_ERR_BAD_COUNT (-2)
#define VIB3_ERR_BAD_POINTER (-3)
#define VIB3_ERR_WORKSPACE (-4)
#define VIB3_ERR_FORMAT (-5) /* a .vib3 file or its page layout is not what the reader expects */
#define VIB3_ERR_IO (-6)     /* a .vib3 file could not be opened or mapped */
#define VIB3_ERR_NOT_RESIDENT (-7) /* a page of a page table has no device address yet */

/* ------------------------------------------------------------------------------------------
 * Reference-compatible launchers: same names, argument order and meaning as cuda_ffi.rs.
 * ---------------------------------------------------------------------------------------- */

/* cuda_ffi.rs:165 (kernels.cu:111, :1043): out_f16[m] = sum_k x_f16[k]*(q-8)*scale_f16.
 * The reference GPU kernel decodes these scales as FP16 (kernels.cu:45, :140). */
int vib3_launch_partial_matmul_int4(const void *input, const void *weight_packed,
                                    const void *scales, void *output, int k, int m_slice,
                                    int group_size, void *stream);

/* cuda_ffi.rs:312 (kernels.cu:175, :1202): same with an f32 input vector. */
int vib3_launch_partial_matmul_int4_f32(const void *input, const void *weight,
                                        const void *scales, void *output, int k, int m_slice,
                                        int group_size, void *stream);

/* cuda_ffi.rs:344 (kernels.cu:279, :1278): out_f16[m] = silu(gate.x) * (up.x), f32 input,
 * FP16 scales. One launch; the two GEMVs and SwiGLU are fused. */
int vib3_launch_fused_swiglu_int4_f32(const void *input, const void *up_weight,
                                      const void *up_scales, const void *gate_weight,
                                      const void *gate_scales, void *output, int k, int m_slice,
                                      int group_size, void *stream);

/* cuda_ffi.rs:186 (kernels.cu:772): out_f16[i] = silu(a[i]) * b[i] for f16 a, b. Argument
 * names follow the reference declaration; the Rust caller passes the gate result first
 * (kernels.rs:283). */
int vib3_launch_silu_mul(const void *up_result, const void *gate_result, void *output, int dim,
                         void *stream);

/* cuda_ffi.rs:202 (kernels.cu:803): out_f32[i] += weight * f32(expert_f16[i]). */
int vib3_launch_weighted_accumulate_f32(void *output, const void *expert_output, float weight,
                                        int dim, void *stream);

/* cuda_ffi.rs:212 (kernels.cu:2092, called from kernels.rs:2051 with the same five
 * arguments): out_f32[i] += weight * expert_f32[i]. */
int vib3_launch_weighted_accumulate_f32_f32(void *output, const void *expert_output,
                                            float weight, int dim, void *stream);

/* cuda_ffi.rs:194 (kernels.cu:788, :1108; kernels.rs:1959): f16 accumulator,
 * out_f16[i] = f16(f32(out_f16[i]) + weight * f32(expert_f16[i])). */
int vib3_launch_weighted_accumulate(void *output, const void *expert_output, float weight,
                                    int dim, void *stream);

/* cuda_ffi.rs:222: out_f32[i] += dev_weight[0] * f32(expert_f16[i]) with the weight read
 * from device memory (no host sync for a router weight). The reference declares this entry
 * point but kernels.cu does not define it; this library does, with the declared meaning. */
int vib3_launch_weighted_accumulate_f32_dev_scalar(void *output, const void *expert_output,
                                                   const void *dev_weight, int dim,
                                                   void *stream);

/* cuda_ffi.rs:267 (kernels.cu:829, :1143): scores[e] = sum_d h_f16[d] * W_f16[e][d] in f32,
 * the GEMV of the reference's GPU router branch (gpu_run_router, kernels.rs:2445-2465); the
 * host does the top-k on the copied scores. One workgroup per expert row (any D, any E). */
int vib3_launch_router_gemv(const void *hidden_state, const void *router_weights, float *scores,
                            int hidden_dim, int num_experts, void *stream);

/* cuda_ffi.rs:369 (kernels.cu:665, :1477): scores[e] = sum_d h_f32[d] * W_f16[e][d]. */
int vib3_launch_router_gemv_f32(const void *hidden_state, const void *router_weights,
                                float *scores, int hidden_dim, int num_experts, void *stream);

/* cuda_ffi.rs:379 (kernels.cu:4075): router GEMV (f32 h, f16 W) + scoring + top-k on device,
 * two launches like the reference. scoring_mode 0: softmax over the top-k of the raw scores;
 * 1: sigmoid (+bias for selection only), normalised, times scaling_factor. Works for any
 * num_experts <= 4096 (the reference kernel needs a power of two). */
int vib3_launch_router_topk(const void *hidden_state, const void *router_weights,
                            float *scores_buf, const float *bias, uint16_t *out_ids,
                            float *out_weights, int hidden_dim, int num_experts, int top_k,
                            int scoring_mode, float scaling_factor, void *stream);

/* cuda_ffi.rs:292 (kernels.cu:921, :1178): out_f32[d] = x[d] * inv_rms * f32(w_f16[d]),
 * inv_rms = 1 / sqrt(sum(x^2) / dim + eps), x f32 (the pre-MoE norm, engine.rs:5072). */
int vib3_launch_rms_norm_f32(const void *input, void *output, const void *weight, int hidden_dim,
                             float eps, void *stream);

/* cuda_ffi.rs:302 (kernels.cu:959): the same, output rounded to f16. */
int vib3_launch_rms_norm_f32_to_f16(const void *input, void *output, const void *weight,
                                    int hidden_dim, float eps, void *stream);

/* cuda_ffi.rs:260 (kernels.cu:817, :1132): accumulator_f32[i] += layer_output_f32[i] (the
 * residual add after the MoE sublayer, engine.rs:5302). */
int vib3_launch_residual_add_f32_f32(void *accumulator, const void *layer_output, int dim,
                                     void *stream);

/* cuda_ffi.rs:233 (kernels.cu:2106): out_f32[i] += sigmoid(gate_dev[0]) * f32(expert_f16[i])
 * (the shared expert's sigmoid gate, engine.rs:6392-6425). */
int vib3_launch_sigmoid_gated_accumulate_f32(void *output, const void *expert_output,
                                             const void *gate_dev, int dim, void *stream);

/* ------------------------------------------------------------------------------------------
 * Additive launchers (no counterpart in cuda_ffi.rs): explicit dtypes, page layout, group
 * size and scale dtype, so one library serves the CPU-fallback semantics (BF16 scales,
 * kernels.rs:2789) and the reference GPU semantics (FP16 scales, kernels.cu:45).
 * ---------------------------------------------------------------------------------------- */

/* partial_matmul (kernels.rs:25) on one INT4 page: output[m] = page . input.
 * input_dtype: F32/F16/BF16; output_dtype: F32/F16; scale_dtype: F16/BF16. */
int vib3_launch_partial_matmul_int4_ex(const void *input, int input_dtype,
                                       const void *weight_page, void *output, int output_dtype,
                                       int k, int m_slice, int group_size, int scale_dtype,
                                       void *stream);

/* partial_swiglu (kernels.rs:162) on one up page and one gate page, fused in one launch:
 * output[m] = silu(gate . input) * (up . input). */
int vib3_launch_partial_swiglu_int4_ex(const void *input, int input_dtype, const void *up_page,
                                       const void *gate_page, void *output, int output_dtype,
                                       int k, int m_slice, int group_size, int scale_dtype,
                                       void *stream);

/* run_router_with_scoring_and_bias (kernels.rs:2307) on device: logits with
 * hidden/weight dtypes of choice, optional f32 bias (selection only), optional normalisation.
 * Two launches (logits, selection). workspace: at least vib3_router_workspace_bytes(num_experts)
 * bytes of scratch. scores_out may be NULL. */
size_t vib3_router_workspace_bytes(int num_experts);
int vib3_launch_router_topk_ex(const void *hidden, int hidden_dtype, const void *router_weights,
                               int weight_dtype, const float *bias, int hidden_dim,
                               int num_experts, int top_k, int scoring_mode,
                               float scaling_factor, int normalize, float *scores_out,
                               uint16_t *out_ids, float *out_weights, void *workspace,
                               void *stream);

/* ------------------------------------------------------------------------------------------
 * Fused MoE layer for batch-1 decode over page-indexed INT4 experts: router -> device ids and
 * weights -> page-table lookup -> fused gate/up GEMV + SwiGLU -> down GEMV with the weighted
 * sum over experts in its epilogue. Three launches (router logits; top-k selection + gate/up;
 * down), no host synchronisation, no atomics, deterministic.
 * Generalises vib3_launch_moe_experts_fused_gpu (cuda_ffi.rs:831, kernels.cu:5868): any number
 * of pages per matrix, INT4 instead of NVFP4, shared experts in the same launches.
 * ---------------------------------------------------------------------------------------- */

#define VIB3_MOE_F32_INTERMEDIATE 1 /* keep h and the down outputs in f32 (no f16 rounding) */
/* Test only: the fused router's bounded wait looks for a tag that no workgroup publishes and
 * gives up after 64 polls, so vib3_moe_int4_layer_status reports 1. Every kernel still exits
 * normally; the routing of such a launch is meaningless. */
#define VIB3_MOE_TEST_ROUTER_TIMEOUT 0x100
/* RMSNorm and shared-expert gates in a prologue kernel of their own instead of inside the
 * gate/up kernel (same results bit for bit; for tests and timing). */
#define VIB3_MOE_SEPARATE_PROLOGUE 0x200

typedef struct vib3_moe_int4_layer {
    /* activation: x[hidden] */
    const void *x;
    int x_dtype;
    int hidden; /* k of gate/up, rows of down */
    int inter;  /* rows of gate/up, k of down */
    int group_size;
    int scale_dtype;
    /* router; when router_w is NULL the experts come from in_ids / in_weights (device) */
    const void *router_w; /* [num_experts][hidden] */
    int router_w_dtype;
    const float *router_bias; /* [num_experts] or NULL */
    int num_experts;
    int top_k;
    int scoring_mode;
    float scaling_factor;
    int normalize;
    const uint16_t *in_ids;
    const float *in_weights;
    /* page tables (device): table[(expert * 3 + segment) * max_pages + page] = page address,
     * segment 0 = up, 1 = gate, 2 = down (types.rs:200 PageId.segment). Page p of a segment
     * holds rows [p * rows_per_page[seg], ...) of that matrix; the last page may be short. */
    const uint64_t *page_table;
    const uint64_t *shared_page_table; /* [num_shared][3][max_pages] or NULL */
    int num_shared;
    int max_pages;
    int rows_per_page[3];
    int flags;
    /* outputs */
    float *out;           /* [hidden] f32, overwritten: sum_j w_j * expert_j(x) + shared */
    uint16_t *out_ids;    /* [top_k] or NULL */
    float *out_weights;   /* [top_k] or NULL */
    float *out_scores;    /* [num_experts] raw logits or NULL */
    void *workspace;      /* vib3_moe_int4_workspace_bytes() bytes of scratch */
    size_t workspace_bytes;
    /* Either side of the sublayer (engine.rs:5064-5307); zero-initialised fields leave the
     * layer as above. norm_weight (f16 [hidden]): x is the f32 residual stream and the router
     * and experts read RMSNorm(x) (vib3_launch_rms_norm_f32's arithmetic, norm_eps).
     * residual (f32 [hidden]): out = residual + sublayer (may alias out).
     * shared_gate (f16 [num_shared][hidden]): shared expert s is weighted by
     * sigmoid(x_normed . shared_gate[s]) instead of 1.0 (engine.rs:6392-6425). */
    const void *norm_weight;
    float norm_eps;
    const float *residual;
    const void *shared_gate;
} vib3_moe_int4_layer;

/* Workspace bytes for `layer`. Zero a new workspace once before its first launch
 * (vib3_hip_zero): the fused router publishes logits there under tags (0 is never a tag). The
 * tag word also lives in the workspace and advances on the device at the end of every launch,
 * so a launch captured in a HIP graph gets a fresh tag on every replay. One workspace serves
 * one launch at a time: launches sharing a workspace must be ordered (one stream). */
size_t vib3_moe_int4_workspace_bytes(const vib3_moe_int4_layer *layer);

/* Status word of the layer's workspace: 1 when a launch's bounded router wait gave up since
 * the last clear (its routing is then not trustworthy), else 0; negative on an argument error.
 * Synchronises `stream` to read it; clear != 0 resets it to 0. With layer->workspace NULL it
 * reads the status of vib3_launch_moe_int4_layer_noalloc calls on the current device.
 * No reference counterpart. */
int vib3_moe_int4_layer_status(const vib3_moe_int4_layer *layer, int clear, void *stream);

/* vib3_launch_moe_int4_layer without a caller workspace and without any allocation: the
 * layer's scratch is a fixed 256 KiB device array of the library (one per GPU, held until the
 * process ends); layer->workspace / workspace_bytes are ignored. A shape whose workspace
 * (vib3_moe_int4_workspace_bytes plus 4 KiB) exceeds 256 KiB returns VIB3_ERR_WORKSPACE
 * (c2: ~45 KiB; c1: ~60 KiB). All calls on one GPU share that scratch: calls that overlap in
 * time on one GPU (two streams, two threads) race and must not be issued; calls ordered on
 * one stream, also under graph capture and replay, are safe. Same kernels and results as
 * vib3_launch_moe_int4_layer. No counterpart in the reference: for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc). */
int vib3_launch_moe_int4_layer_noalloc(const vib3_moe_int4_layer *layer, void *stream);

/* 1 when the layer computes the router logits and top-k inside its gate/up kernel (up to 512
 * experts), 0 when the router runs as launches of its own. */
int vib3_moe_int4_router_fused(const vib3_moe_int4_layer *layer);
int vib3_launch_moe_int4_layer(const vib3_moe_int4_layer *layer, void *stream);

/* One stage of the same layer: 0 = router (logits and, when separate, selection), 1 = fused
 * gate/up + SwiGLU, 2 = down + weighted combine. A stage reads what the earlier stages of a
 * previous call left in the workspace; for timing each stage's kernels on their own. */
int vib3_launch_moe_int4_layer_stage(const vib3_moe_int4_layer *layer, int stage, void *stream);

/* ------------------------------------------------------------------------------------------
 * The reference's sync-free fused MoE over NVFP4 pages (kernels.cu:5650-5990): FP4 activation
 * (split-half E2M1, E8M0 per 32) times up/gate pages -> SwiGLU -> FP4 h -> down pages ->
 * layer_output += w * down, for up to 8 experts. Pages hold tiled split-half E2M1 data
 * (16 rows x 64 columns per 512-byte tile, after vib3_launch_repack_weights_inplace and
 * vib3_launch_repack_row_to_tiled) followed by [rows][k/32] 2-byte scales whose exponent byte
 * (s >> 7 & 0xff, a bf16's) is the E8M0 block scale (kernels.cu:5404-5411). Sums are exact
 * (f64) and rounded once to f32, so results do not depend on launch order. Shapes: k_in and
 * m_mid multiples of 128, m_out of 16, k_mid == m_mid, and each kernel's LDS within 64 KB:
 * about k_in <= 15360 and num_experts * m_mid <= 24576 (VIB3_ERR_UNSUPPORTED otherwise). A slot whose id is
 * >= num_experts_total or whose table entry is 0 contributes nothing.
 * ---------------------------------------------------------------------------------------- */

/* cuda_ffi.rs:625 (kernels.cu:3193-3266): f32 input[K] -> act_fp4[K/2] split-half E2M1
 * (16-byte aligned) and act_scales[K/32] E8M0 = round(log2 amax) - 2 + 127 per 32 values. */
int vib3_launch_quantize_activation_fp4(const void *input, void *act_fp4, void *act_scales,
                                        int K, void *stream);
/* cuda_ffi.rs:781 (kernels.cu:6585-6727, kernels.rs:1641): RMSNorm of the f32 hidden state
 * with f16 weights, quantized as vib3_launch_quantize_activation_fp4, in one launch;
 * opt_f16_out (or NULL) receives the normalised values as f16. The sum of squares follows the
 * reference's order; the inverse RMS is the correctly rounded 1/sqrtf where the reference
 * uses the approximate rsqrtf. K a multiple of 32 (VIB3_ERR_UNSUPPORTED otherwise; the
 * reference covers K/64 whole tiles). */
int vib3_launch_fused_rms_norm_quantize_fp4(const void *input, const void *norm_weight,
                                            void *act_fp4, void *act_scales, void *opt_f16_out,
                                            int K, float eps, void *stream);

/* cuda_ffi.rs:770 (kernels.cu:5252): the same. */
int vib3_launch_quantize_activation_fp4_fast(const void *input, void *act_fp4,
                                             void *act_scales, int K, void *stream);

/* cuda_ffi.rs:1026 (kernels.cu:6507): allocate the fused MoE's intermediate buffer (FP4 h of 8
 * experts) on the current device. Without it, the first launch of the entry points below
 * that take no workspace allocates it (the reference's ensure_moe_bufs, kernels.cu:5675);
 * call it before graph capture, where a launch that would allocate returns
 * VIB3_ERR_WORKSPACE instead. Those entry points share this one buffer per device: launches
 * on one device must be ordered (one stream at a time); for concurrent streams use the _ws
 * forms, each with a workspace of its own. */
int vib3_moe_prewarm_gpu_bufs(int m_mid, int k_mid);

/* Bytes of the caller workspace of the _ws forms below (256-byte aligned device memory). No
 * reference counterpart. */
size_t vib3_moe_experts_fused_workspace_bytes(int m_mid);

/* cuda_ffi.rs:809 (kernels.cu:5650): host arrays of device pointers per expert (data and
 * scales of up, gate, down) and host routing weights; layer_output accumulated (+=). */
int vib3_launch_moe_experts_fused(const void *act_fp4, const void *act_scales,
                                  const void *const *up_weight_ptrs,
                                  const void *const *up_scale_ptrs,
                                  const void *const *gate_weight_ptrs,
                                  const void *const *gate_scale_ptrs,
                                  const void *const *down_weight_ptrs,
                                  const void *const *down_scale_ptrs,
                                  const float *expert_weights_host, int num_experts, int K_in,
                                  int M_mid, int K_mid, int M_out, float *layer_output,
                                  void *stream);

/* cuda_ffi.rs:831 (kernels.cu:5868): the same from a device page table
 * page_table[(layer * num_experts_total + id) * 3 + seg] (engine.rs:1236-1299; seg 0 up,
 * 1 gate, 2 down; scales at page + K/2 * rows) and device ids / weights of num_active experts. */
int vib3_launch_moe_experts_fused_gpu(const void *act_fp4, const void *act_scales,
                                      const uint64_t *page_table, const uint16_t *expert_ids,
                                      const float *expert_weights, int layer,
                                      int num_experts_total, int num_active, int K_in, int M_mid,
                                      int K_mid, int M_out, float *layer_output, void *stream);

/* vib3_launch_moe_experts_fused[_gpu] with the intermediate buffer in the caller's workspace
 * (vib3_moe_experts_fused_workspace_bytes(M_mid) bytes, 256-byte aligned): reentrant, so
 * launches on different streams with different workspaces may overlap. No reference
 * counterpart (additive). */
int vib3_launch_moe_experts_fused_ws(const void *act_fp4, const void *act_scales,
                                     const void *const *up_weight_ptrs,
                                     const void *const *up_scale_ptrs,
                                     const void *const *gate_weight_ptrs,
                                     const void *const *gate_scale_ptrs,
                                     const void *const *down_weight_ptrs,
                                     const void *const *down_scale_ptrs,
                                     const float *expert_weights_host, int num_experts, int K_in,
                                     int M_mid, int K_mid, int M_out, float *layer_output,
                                     void *workspace, size_t workspace_bytes, void *stream);
int vib3_launch_moe_experts_fused_gpu_ws(const void *act_fp4, const void *act_scales,
                                         const uint64_t *page_table, const uint16_t *expert_ids,
                                         const float *expert_weights, int layer,
                                         int num_experts_total, int num_active, int K_in,
                                         int M_mid, int K_mid, int M_out, float *layer_output,
                                         void *workspace, size_t workspace_bytes, void *stream);

/* cuda_ffi.rs:671 (kernels.cu:4708): one expert over tiled split-half pages: up and gate
 * GEMVs, SwiGLU, FP4 h, down GEMV, layer_output += expert_weight * down (the fused pipeline
 * above with one expert; same buffer rule). */
int vib3_launch_expert_batched(const void *act_fp4, const void *act_scales,
                               const void *up_weight, const void *up_scales,
                               const void *gate_weight, const void *gate_scales,
                               const void *down_weight, const void *down_scales,
                               float *layer_output, float expert_weight, int K_in, int M_mid,
                               int K_mid, int M_out, void *stream);

/* cuda_ffi.rs:851 (kernels.cu:6017-6154): f16 weights [M][K] -> row-major split-half E2M1
 * codes [M][K/2] and bf16 scales [M][K/32] = 2^(e - 127) with e the E8M0 of each 32-value
 * group (the activation quantizer's rule). K % 32 == 0. */
int vib3_launch_fp16_to_nvfp4_weight(const void *input, void *out_data, void *out_scales, int M,
                                     int K, void *stream);

/* ------------------------------------------------------------------------------------------
 * Per-page NVFP4 GEMVs (fp4_pages.hip), the reference's launchers for NVFP4 experts spread
 * over several pages (engine.rs:5960-6226). A page is [M][K/2] code bytes then [M][K/32]
 * 2-byte scales. K % 32 == 0 (tiled: K % 64 == 0, M % 16 == 0), data 16-byte aligned.
 * Block-scaled (E2M1 x FP4 activation): exact group sums in f64, one rounding to f32 output;
 * the scale's exponent byte is the E8M0 (gemv_scalar: its bf16 value).
 * ---------------------------------------------------------------------------------------- */

/* cuda_ffi.rs:634 (kernels.cu:3752): row-major split-half weights, pre-quantized activation. */
int vib3_launch_gemv_mma_nvfp4_preq(const void *act_fp4, const void *act_scales,
                                    const void *weight_packed, const void *scales, void *output,
                                    int K, int M_slice, void *stream);
/* cuda_ffi.rs:690 (kernels.cu:5229): the same. */
int vib3_launch_gemv_mma_nvfp4_preq_fast(const void *act_fp4, const void *act_scales,
                                         const void *weight_packed, const void *scales,
                                         void *output, int K, int M_slice, void *stream);
/* cuda_ffi.rs:646 (kernels.cu:3853, :3789): output = (g * sigmoid(g)) * u of the up and gate
 * GEMVs above, f32. */
int vib3_launch_fused_swiglu_mma_nvfp4_preq(const void *act_fp4, const void *act_scales,
                                            const void *up_weight, const void *up_scales,
                                            const void *gate_weight, const void *gate_scales,
                                            void *output, int K, int M_slice, void *stream);
/* cuda_ffi.rs:793 (kernels.cu:5267): the same. */
int vib3_launch_fused_swiglu_mma_nvfp4_preq_fast(const void *act_fp4, const void *act_scales,
                                                 const void *up_weight, const void *up_scales,
                                                 const void *gate_weight, const void *gate_scales,
                                                 void *output, int K, int M_slice, void *stream);
/* cuda_ffi.rs:729 (kernels.cu:4359): tiled split-half weights. */
int vib3_launch_gemv_mma_nvfp4_tiled(const void *act_fp4, const void *act_scales,
                                     const void *weight, const void *scales, void *output, int K,
                                     int M_slice, void *stream);
/* cuda_ffi.rs:703 (kernels.cu:4520): row-major split-half weights, scales read as bf16 values. */
int vib3_launch_gemv_scalar_nvfp4(const void *act_fp4, const void *act_scales,
                                  const void *weight_packed, const void *scales, void *output,
                                  int K, int M_slice, void *stream);
/* cuda_ffi.rs:599 / :611 (kernels.cu:3676, :3807): f32 input quantized to FP4 in the kernel
 * (vib3_launch_quantize_activation_fp4's rule), sequential-nibble weights. */
int vib3_launch_gemv_mma_nvfp4(const void *input, const void *weight_packed, const void *scales,
                               void *output, int K, int M_slice, void *stream);
int vib3_launch_fused_swiglu_mma_nvfp4(const void *input, const void *up_weight,
                                       const void *up_scales, const void *gate_weight,
                                       const void *gate_scales, void *output, int K,
                                       int M_slice, void *stream);

/* Scalar NVFP4 GEMVs (cuda_ffi.rs:532-597; kernels.cu:446, :512, :598, :1957, :2035): f32 (or
 * f16: _fp16in) input times sequential-nibble E2M1 weights times the bf16 block scale
 * (block_size a power-of-two multiple of 32), accumulated in f32; f16 output (or f32: _f32out);
 * SwiGLU output silu(g) * u with silu(g) = g / (1 + e^-g). */
int vib3_launch_partial_matmul_nvfp4(const void *input, const void *weight_packed,
                                     const void *scales, void *output, int K, int M_slice,
                                     int block_size, void *stream);
int vib3_launch_partial_matmul_nvfp4_f32out(const void *input, const void *weight_packed,
                                            const void *scales, void *output, int K, int M_slice,
                                            int block_size, void *stream);
int vib3_launch_partial_matmul_nvfp4_fp16in(const void *input, const void *weight_packed,
                                            const void *scales, void *output, int K, int M_slice,
                                            int block_size, void *stream);
int vib3_launch_fused_swiglu_nvfp4(const void *input, const void *up_weight,
                                   const void *up_scales, const void *gate_weight,
                                   const void *gate_scales, void *output, int K, int M_slice,
                                   int block_size, void *stream);
int vib3_launch_fused_swiglu_nvfp4_f32out(const void *input, const void *up_weight,
                                          const void *up_scales, const void *gate_weight,
                                          const void *gate_scales, void *output, int K,
                                          int M_slice, int block_size, void *stream);

/* cuda_ffi.rs:662 (kernels.cu:4132-4183): sequential nibble order -> split-half, in place, per
 * 16-byte block of the page's data (a partial last block is left as it is). */
int vib3_launch_repack_weights_inplace(void *weight_data_ptr, long long weight_data_bytes,
                                       void *stream);

/* cuda_ffi.rs:718 (kernels.cu:4227-4262): row-major split-half [M][K/2] -> tiled, through
 * temp_buf (M*K/2 bytes), then copied back. M % 16 == 0, K % 64 == 0. */
int vib3_launch_repack_row_to_tiled(void *weight_data_ptr, void *temp_buf, int M, int K,
                                    void *stream);

/* ------------------------------------------------------------------------------------------
 * Batched decode over MXFP4 experts (no counterpart in cuda_ffi.rs): T tokens, top_k picks
 * each, grouped per expert and run as a grouped GEMM on the CDNA4 matrix cores.
 * Per token t: h = f16(silu(gate_e . x_t) * (up_e . x_t)), d_j = f16(down_e . h),
 * out[t] = bf16(sum_j w[t,j] * d_j) in pick order: the per-token composition of engine.rs
 * (execute_expert, :5801-6306) with MXFP4 weights, E2M1 codes (kernels.cu:438-441, low nibble =
 * even k) times E8M0 scales 2^(e-127) per 32 along k (kernels.cu:2770-2777).
 * MXFP4 page: [rows x k/2] code bytes, then [rows x k/32] E8M0 bytes.
 * ---------------------------------------------------------------------------------------- */
typedef struct vib3_moe_mxfp4_batch {
    const void *x;           /* [tokens][hidden] bf16, 16-byte aligned */
    int tokens;
    int hidden;              /* multiple of 256 */
    int inter;               /* multiple of 256 */
    int num_experts;         /* <= 4096 */
    int top_k;               /* tokens * top_k <= 4096 */
    const uint16_t *ids;     /* [tokens][top_k] device; ids >= num_experts are skipped */
    const float *weights;    /* [tokens][top_k] device */
    const uint64_t *page_table; /* [num_experts][3] device: up, gate, down MXFP4 pages */
    void *out;               /* [tokens][hidden] bf16 */
    void *workspace;         /* vib3_moe_mxfp4_workspace_bytes() bytes, 256-byte aligned */
    size_t workspace_bytes;
} vib3_moe_mxfp4_batch;

size_t vib3_moe_mxfp4_workspace_bytes(const vib3_moe_mxfp4_batch *batch);
int vib3_launch_moe_mxfp4_batched(const vib3_moe_mxfp4_batch *batch, void *stream);

/* ------------------------------------------------------------------------------------------
 * The .vib3 model file (host side; format.rs). The file is memory-mapped read-only; page data
 * is returned as host pointers into the mapping, for the caller to upload where its page pool
 * lives. vib3_build_page_table then writes the fused layer's page table from the catalog.
 * ---------------------------------------------------------------------------------------- */

typedef struct vib3_file vib3_file; /* opaque: the mapping plus the parsed catalog */

/* Header summary (format.rs:50-92 Vib3Header). expert_dtype / shared_dtype use the reference's
 * DType codes (types.rs:633: 0 FP16, 1 BF16, 5 INT4, 7 NVFP4, ...). */
typedef struct vib3_file_info {
    uint32_t num_layers, num_experts, num_active_experts, hidden_dim, expert_hidden_dim;
    uint8_t expert_dtype, shared_dtype;
    uint32_t page_count;
    uint64_t page_data_offset, page_data_size;
} vib3_file_info;

/* One page catalog entry (format.rs:101-125 PageCatalogEntry) and its index in the catalog. */
typedef struct vib3_page_entry {
    uint16_t layer, expert, segment, page_idx; /* types.rs:201 PageId */
    uint64_t file_offset;
    uint32_t compressed_size, raw_size;
    uint16_t row_start, row_count, col_start, col_count;
    uint8_t compression, flags; /* compression: 0 none, 1 LZ4, 2 zstd (format.rs:43-45) */
    uint32_t catalog_index;
} vib3_page_entry;

/* format.rs:241 Vib3File::open: magic/version checked, catalog and expert index parsed. */
int vib3_file_open(const char *path, vib3_file **out);
void vib3_file_close(vib3_file *file);
int vib3_file_get_info(const vib3_file *file, vib3_file_info *info);
/* The model metadata section (JSON, format.rs:263-272), not NUL-terminated. */
int vib3_file_metadata(const vib3_file *file, const char **json, size_t *len);
/* Catalog entry `index` (format.rs:355). */
int vib3_file_page(const vib3_file *file, uint32_t index, vib3_page_entry *entry);
/* format.rs:371 pages_for_expert: the entries of (layer, expert) in catalog order (segment,
 * then page_idx); *count = their number (at most max_entries are written). expert 0xFFFF is
 * the layer's shared tensors (router segment 3, norms, shared experts 14/15/16, gate 26). */
int vib3_file_expert_pages(const vib3_file *file, uint16_t layer, uint16_t expert,
                           vib3_page_entry *out, int max_entries, int *count);
/* format.rs:501 read_page_sync for an uncompressed page: a pointer into the mapping and its
 * size. Compressed pages return VIB3_ERR_UNSUPPORTED (no LZ4/zstd codec in this build). */
int vib3_file_page_data(const vib3_file *file, uint32_t index, const void **data, size_t *size);
/* format.rs:501 read_page_sync: the page's bytes into a host buffer of `capacity` bytes,
 * LZ4 pages (lz4_flex size-prepended blocks) decompressed; zstd pages return
 * VIB3_ERR_UNSUPPORTED. *written = the page's raw size. */
int vib3_file_read_page(const vib3_file *file, uint32_t index, void *dst, size_t capacity,
                        size_t *written);

/* The page table of vib3_moe_int4_layer from the catalog (engine.rs:1236-1299, one page per
 * segment there; any number here): for each experts[i] of `layer` and each of its segments
 * segments[0..2] (up, gate, down: {0, 1, 2} for routed experts, {14, 15, 16} for shared ones),
 * table[(i*3 + s)*max_pages + page_idx] = page_addr[catalog index of that page] (where the
 * caller put the page). rows_per_page[s] receives the segment's rows per page. Pages must
 * cover rows [p*rows_per_page, ...) in order, every page but the last full (the converter's
 * layout, convert.rs:1852-1865), and reach rows_required[s] rows (NULL: the file's
 * expert_hidden_dim for up/gate and hidden_dim for down): a truncated segment is
 * VIB3_ERR_FORMAT, a page whose address is 0 VIB3_ERR_NOT_RESIDENT. Host memory in and out. */
int vib3_build_page_table(const vib3_file *file, uint16_t layer, const uint16_t *experts,
                          int num_experts, const uint16_t segments[3],
                          const uint64_t *page_addr, uint64_t *table, int max_pages,
                          int rows_per_page[3], const int *rows_required);

/* One entry of the query planner's plan, query_planner.rs:38-43 ResolvedPage{id, device_ptr,
 * row_start, row_count} with its PageId (types.rs:199-205, repr(C)) spelled out. device_ptr 0:
 * the page is not resident on the device (buffer_manager.rs:775 get_page would fetch it). */
typedef struct vib3_resolved_page {
    uint16_t layer, expert, segment, page_idx;
    uint64_t device_ptr;
    uint16_t row_start, row_count;
} vib3_resolved_page;

/* The same table from the planner's ResolvedPage lists (the pages of one layer, any order):
 * the page of (experts[i], segments[s], page_idx) goes to table[(i*3 + s)*max_pages + page_idx],
 * with the checks of vib3_build_page_table against rows_required[s] (NULL: unchecked). Pages
 * with device_ptr 0 leave their entry 0; their indices in `pages` are written to
 * missing[0..max_missing) in table order (expert, segment, page), *num_missing receives their number and the call
 * returns VIB3_ERR_NOT_RESIDENT: the caller fetches them (get_page) and builds again. The
 * layer must not be launched on such a table. Host memory in and out. */
int vib3_build_page_table_resolved(const vib3_resolved_page *pages, size_t num_pages,
                                   const uint16_t *experts, int num_experts,
                                   const uint16_t segments[3], const int rows_required[3],
                                   uint64_t *table, int max_pages, int rows_per_page[3],
                                   uint32_t *missing, int max_missing, int *num_missing);

/* ------------------------------------------------------------------------------------------
 * Utilities
 * ---------------------------------------------------------------------------------------- */

/* Zero `bytes` of device memory with a fill kernel (safe inside HIP graph capture). */
int vib3_hip_zero(void *ptr, size_t bytes, void *stream);

/* Synthetic data (no reference counterpart): counter-based generator whose spec is restated
 * in the CPU oracle, so host and device produce identical bytes.
 *   bytes:  byte j = (hash(seed, stream, j/8) >> 8*(j%8)) & 0xff for j in [off, off+n)
 *   normal: Irwin-Hall(4) normal * sigma, written as dtype
 *   int4 page: rows [row_start, row_start+rows) of the logical matrix `stream` (k, g). */
int vib3_synth_bytes(void *dst, size_t n, uint64_t seed, uint64_t stream, size_t off,
                     void *hip_stream);
int vib3_synth_normal(void *dst, int dtype, size_t n, uint64_t seed, uint64_t stream,
                      size_t off, float sigma, void *hip_stream);
int vib3_synth_int4_page(void *page, uint64_t seed, uint64_t stream, int k, int group_size,
                         int scale_dtype, float sigma, int row_start, int rows,
                         void *hip_stream);

/* Rows [row_start, row_start + rows) of the logical MXFP4 matrix `stream` (k columns) as one
 * page: code bytes from stream*2, E8M0 bytes 119 + hash % 5 (2^-8 .. 2^-4) from stream*2+1. */
int vib3_synth_mxfp4_page(void *page, uint64_t seed, uint64_t stream, int k, int row_start,
                          int rows, void *hip_stream);

/* Library version string. */
const char *vib3_hip_version(void);

#ifdef __cplusplus
}
#endif
#endif
