/*
 * oracle/cpu_ref.h — CPU restatement of vib3's MoE expert path (TEST INFRASTRUCTURE ONLY).
 *
 * This library is the parity oracle for the HIP kernels in vib3_amd/csrc. It restates, in plain
 * C with sequential fp32 arithmetic (built with -ffp-contract=off so a*b+c is never fused), the
 * CPU fallback of the reference crate (threehundobaud/vic, crate `vib3`):
 *
 *   v3o_matmul_int4_acc      <- src/compute/kernels.rs:2746-2832 (cpu_matmul_int4_grouped)
 *   v3o_partial_matmul_int4  <- src/compute/kernels.rs:25-67, :2733 (partial_matmul, INT4 arm)
 *   v3o_swiglu_int4_acc      <- src/compute/kernels.rs:2932-3054 (cpu_swiglu_int4)
 *   v3o_partial_swiglu_int4  <- src/compute/kernels.rs:162-203 (partial_swiglu, INT4 arm)
 *   v3o_weighted_accumulate_f32 <- src/compute/kernels.rs:2000-2036
 *   v3o_weighted_accumulate_f16 <- src/compute/kernels.rs:1959-1996
 *   v3o_router               <- src/compute/kernels.rs:2307-2440 (run_router_with_scoring_and_bias)
 *   v3o_quantize_int4        <- src/compute/kernels.rs:3778-3831 (quantize_weights_to_int4)
 *   v3o_dequantize_int4      <- src/compute/kernels.rs:3866-3927 (dequantize_int4_to_f32)
 *   v3o_moe_layer            <- src/runtime/engine.rs:5801-6306 (execute_expert),
 *                               :6317-6456 (execute_shared_expert, weight 1.0 without gate)
 *   v3o_moe_layer_w          <- the same with the shared expert's sigmoid gate, engine.rs:6392-6451
 *   v3o_rms_norm_f32         <- cuda/src/kernels.cu:921-955 (vib3_rms_norm_f32; no CPU body exists)
 *   v3o_residual_add_f32     <- cuda/src/kernels.cu:817 (vib3_residual_add_f32_f32_kernel)
 *   v3o_linear_row_f16       <- src/compute/kernels.rs:3630-3640 (linear_projection_f32_to_f32)
 *   v3o_mxfp4_*              <- cuda/src/kernels.cu:438-441 (E2M1 table), :2770-2777 (E8M0)
 *   v3o_fp4_quantize_act     <- cuda/src/kernels.cu:3193-3240 (+ compute_e8m0 :2759-2768)
 *   v3o_fused_rms_norm_quantize_fp4, v3o_fp4_norm_inv
 *                            <- cuda/src/kernels.cu:6585-6702 (sum order kept; rsqrtf replaced
 *                               by the correctly rounded 1 / sqrtf)
 *   v3o_nvfp4_matvec         <- cuda/src/kernels.cu:5357-5449 (tiled split-half MMA GEMV)
 *   v3o_moe_experts_fused    <- cuda/src/kernels.cu:5650-5834, :5868-5990 (fused NVFP4 MoE)
 *   v3o_fp4_split_half / v3o_fp4_to_tiled <- cuda/src/kernels.cu:4132-4160, :4190-4225
 *   v3o_quantize_weights_to_nvfp4 <- src/compute/kernels.rs:4085-4170
 *   v3o_quantize_half_to_nvfp4    <- src/compute/kernels.rs:4172-4188
 *   v3o_convert_int4_to_nvfp4     <- src/compute/kernels.rs:3937-4060
 *   v3o_fp16_to_nvfp4_weight      <- cuda/src/kernels.cu:6017-6128
 *   v3o_nvfp4_page_matvec / _swiglu <- cuda/src/kernels.cu:3276-3385, :3739-3905, :4265-4540
 *   v3o_synth_*              synthetic-data generator spec shared with vib3_amd/csrc/synth.hip
 *
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load this library,
 * and only as the checker / the timed CPU baseline. The product path never calls it.
 *
 * Parity pins (what checks each function independently of its own formula) are listed in
 * tests/test_oracle.py: the reference's known-answer tests, f64 brute force on small shapes,
 * closed forms and invariants. Functions whose rounding points only a restatement can fix
 * (sequential fp32 sum order, f16 output rounding, libm expf) are pinned up to those points.
 */
#ifndef VIB3_ORACLE_CPU_REF_H
#define VIB3_ORACLE_CPU_REF_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* dtype codes shared with include/vib3_hip.h */
enum { V3O_F32 = 0, V3O_F16 = 1, V3O_BF16 = 2 };

/* IEEE conversions with round-to-nearest-even, the semantics of `half` 2.7.1
 * (Cargo.lock:885-886) used by the reference for f16/bf16 <-> f32. */
uint16_t v3o_f32_to_f16(float f);
float v3o_f16_to_f32(uint16_t h);
uint16_t v3o_f32_to_bf16(float f);
float v3o_bf16_to_f32(uint16_t b);
/* convert n elements of dtype `dt` at src to f32 */
void v3o_to_f32(const void *src, int dt, size_t n, float *dst);

/* Number of worker threads used by the row-parallel functions when nthreads <= 0. */
int v3o_default_threads(void);

/* INT4 page: [m x ceil(k/2)] packed nibbles (low nibble = even column, stored q = code+8),
 * then [m x ceil(k/g)] little-endian 2-byte scales (scale_dt = V3O_BF16 or V3O_F16).
 * acc[row] = sum_k x[k] * LUT_g[q]  with LUT_g[q] = (q-8)*s_g  (sequential fp32, k order).
 * Invalid scale (non-finite or <= 0) decodes as 1/8 (kernels.rs:2791-2797). */
void v3o_matmul_int4_acc(const float *x, const uint8_t *page, size_t k, size_t m, size_t g,
                         int scale_dt, float *acc, int nthreads);

/* Public CPU entry of partial_matmul(..., DType::INT4): f16 in, f16 out, g = 32, BF16 scales. */
void v3o_partial_matmul_int4(const uint16_t *x_f16, const uint8_t *page, uint16_t *out_f16,
                             size_t k, size_t m);

/* h[row] = silu(gate_acc) * up_acc (fp32, before the f16 rounding of the reference). */
void v3o_swiglu_int4_acc(const float *x, const uint8_t *up_page, const uint8_t *gate_page,
                         size_t k, size_t m, size_t g, int scale_dt, float *h, int nthreads);

/* Public CPU entry of partial_swiglu(..., DType::INT4): f16 in/out, g = 32, BF16 scales. */
void v3o_partial_swiglu_int4(const uint16_t *x_f16, const uint8_t *up_page,
                             const uint8_t *gate_page, uint16_t *out_f16, size_t k, size_t m);

/* out[i] += w * f32(expert_f16[i]) */
void v3o_weighted_accumulate_f32(float *out, const uint16_t *expert_f16, float w, size_t n);
/* out_f16[i] = f16(f32(out_f16[i]) + w * f32(expert_f16[i])) */
void v3o_weighted_accumulate_f16(uint16_t *out, const uint16_t *expert_f16, float w, size_t n);

/* Router: scores[e] = sum_d x[d]*W[e][d] (sequential fp32), then
 * mode 0 (softmax): stable sort desc on scores, keep k, softmax over the k;
 * mode 1 (sigmoid): sel = sigmoid + bias, stable sort desc, keep k, weight = sigmoid,
 *                   normalise if sum > 1e-20 and `normalize`, then * scaling.
 * W dtype: V3O_F32 / V3O_F16 / V3O_BF16. bias may be NULL. scores_out may be NULL.
 * Returns 0, or -1 for bad arguments. */
int v3o_router(const float *x, const void *w, int w_dt, size_t num_experts, size_t hidden,
               size_t top_k, int mode, float scaling, int normalize, const float *bias,
               uint16_t *ids, float *weights, float *scores_out, int nthreads);

/* Quantizer with the group size as a parameter (the reference fixes g = 32). Scales BF16. */
void v3o_quantize_int4(const float *w, size_t rows, size_t cols, size_t g, uint8_t *out);
void v3o_dequantize_int4(const uint8_t *page, size_t rows, size_t cols, size_t g, int scale_dt,
                         float *out);

/* One expert's matrices: each is a list of pages with a uniform row count per page
 * (the last page may be shorter); each page holds [rows x pk][rows x G x 2] like a
 * vib3 INT4 page (kernels.rs:95-98, convert.rs:1807-1880). */
typedef struct {
    const uint8_t *const *pages; /* npages pointers */
    size_t npages;
    size_t rows_per_page;
} v3o_matrix;

typedef struct {
    v3o_matrix up, gate, down; /* segment 0 = up, 1 = gate, 2 = down (types.rs:200) */
} v3o_expert;

/* MoE layer as the engine composes it: for each selected expert (router order):
 *   h = f16(silu(gate.x) * up.x)  per up/gate page pair into h[row_start..]
 *   d = f16(down . h)             per down page
 *   out += w * d                  (weighted_accumulate_f32)
 * then each shared expert with weight 1.0. out is zeroed first.
 * faithful = 1 keeps the reference's f16 rounding of h and d; 0 keeps them fp32. */
void v3o_moe_layer(const float *x, size_t hidden, size_t inter, size_t g, int scale_dt,
                   const v3o_expert *routed, const uint16_t *ids, const float *weights,
                   size_t top_k, const v3o_expert *shared, size_t n_shared, int faithful,
                   float *out, int nthreads);

/* The same with the shared experts weighted by shared_w[s] (NULL: 1.0). */
void v3o_moe_layer_w(const float *x, size_t hidden, size_t inter, size_t g, int scale_dt,
                     const v3o_expert *routed, const uint16_t *ids, const float *weights,
                     size_t top_k, const v3o_expert *shared, size_t n_shared,
                     const float *shared_w, int faithful, float *out, int nthreads);

/* Either side of the sublayer: RMSNorm (kernels.cu:921), residual add (kernels.cu:817),
 * the shared-expert gate logit (kernels.rs:3630) and its sigmoid (kernels.cu:2114). */
float v3o_inv_rms(const float *x, size_t n, float eps);
void v3o_rms_norm_f32(const float *x, size_t n, const uint16_t *w_f16, float eps, float *out);
void v3o_residual_add_f32(float *acc, const float *lo, size_t n);
float v3o_linear_row_f16(const float *x, const uint16_t *w_f16, size_t n);
float v3o_sigmoid(float g);

/* MXFP4: E2M1 code (low nibble = even k) times E8M0 scale 2^(e-127) per 32 along k. */
float v3o_e2m1(uint8_t code);
float v3o_e8m0(uint8_t e);
/* acc[row] = sum_k x[k] * e2m1(q) * 2^(e-127)  (sequential fp32 over k; each term rounded) */
void v3o_matmul_mxfp4_acc(const float *x, const uint8_t *codes, const uint8_t *scales, size_t k,
                          size_t m, float *acc, int nthreads);

/* Batched MoE over MXFP4 experts (c4), restated per token: pages[e*3 + {0 up, 1 gate, 2 down}]
 * are MXFP4 pages ([rows x k/2] codes, then [rows x k/32] E8M0 bytes); x is [tokens][hidden];
 * picks with ids >= num_experts are skipped; out is [tokens][hidden] bf16. */
void v3o_moe_mxfp4_batched(const float *x, size_t tokens, size_t hidden, size_t inter,
                           const uint8_t *const *pages, size_t num_experts, const uint16_t *ids,
                           const float *weights, size_t top_k, uint16_t *out, int nthreads);

/* ---- NVFP4 fused MoE (split-half E2M1, tiled weights, E8M0 = bf16 scale >> 7) ---- */
uint8_t v3o_fp4_e8m0_of_amax(float amax);
uint8_t v3o_e2m1_rne(float v);
float v3o_exp_cw(float x);
/* x[k] f32 -> codes[ceil(k/32) * 16] split-half, scales[ceil(k/32)] E8M0 */
void v3o_fp4_quantize_act(const float *x, size_t k, uint8_t *codes, uint8_t *scales);
float v3o_fp4_norm_inv(const float *x, size_t k, float eps);
void v3o_fused_rms_norm_quantize_fp4(const float *x, const uint16_t *w_f16, size_t k, float eps,
                                     uint8_t *codes, uint8_t *scales, uint16_t *f16_out);
/* out[m] = f32(exact sum over k of W[r][k] * a[k]); data tiled, scales [m][k/32] 2-byte */
void v3o_nvfp4_matvec(const uint8_t *act_codes, const uint8_t *act_scales, const uint8_t *data,
                      const uint16_t *scales, size_t m, size_t k, float *out);
/* data[e*3 + {0 up, 1 gate, 2 down}], scales likewise; out[m_out] accumulated in place */
void v3o_moe_experts_fused(const uint8_t *act_codes, const uint8_t *act_scales,
                           const uint8_t *const *data, const uint16_t *const *scales,
                           const float *weights, size_t n, size_t k_in, size_t m_mid,
                           size_t m_out, float *out);
void v3o_fp4_split_half(uint8_t *data, size_t nbytes);
void v3o_fp4_to_tiled(const uint8_t *src, uint8_t *dst, size_t m, size_t k);

/* ---- NVFP4 weight quantizers (row-major sequential E2M1, FP16 block scales per 32) ---- */
size_t v3o_nvfp4_page_bytes(size_t rows, size_t cols);
/* kernels.rs:4085 quantize_weights_to_nvfp4: out = [rows x ceil(cols/2)] codes then
 * [rows x ceil(cols/32)] f16 scales (max|w| / 6) */
void v3o_quantize_weights_to_nvfp4(const float *w, size_t rows, size_t cols, uint8_t *out);
/* kernels.rs:4172 / :4183 quantize_{fp16,bf16}_to_nvfp4 (dt = V3O_F16 / V3O_BF16) */
void v3o_quantize_half_to_nvfp4(const uint16_t *w, int dt, size_t rows, size_t cols,
                                uint8_t *out);
/* kernels.rs:3937 convert_int4_to_nvfp4 (INT4 page with BF16 group scales of size g; len =
 * the page's byte length, for the reference's bounds rule) */
void v3o_convert_int4_to_nvfp4(const uint8_t *int4, size_t len, size_t rows, size_t cols,
                               size_t g, uint8_t *out);
/* kernels.cu:6017 vib3_fp16_to_nvfp4_weight: f16 [m][k] -> row-major split-half E2M1 codes
 * [m][k/2] and bf16 scales 2^(e-127) ([m][k/32], E8M0 e in bits 7..14), k a multiple of 32 */
void v3o_fp16_to_nvfp4_weight(const uint16_t *w_f16, size_t m, size_t k, uint8_t *data,
                              uint16_t *scales);
/* f64 matvec of a row-major sequential NVFP4 matrix with full BF16 scales */
void v3o_nvfp4_seq_matvec_f64(const float *x, const uint8_t *data, const uint16_t *scales,
                              size_t m, size_t k, double *out);

/* ---- per-page NVFP4 GEMVs (pre-quantized activation; layout 0 row-major split-half,
 * 1 tiled, 2 row-major sequential; full = 0: weight scale = E8M0 byte of the bf16, 1: the
 * bf16 value) ---- */
void v3o_nvfp4_page_matvec(const uint8_t *act_codes, const uint8_t *act_scales,
                           const uint8_t *data, const uint16_t *scales, size_t m, size_t k,
                           int layout, int full, float *out);
void v3o_nvfp4_page_swiglu(const uint8_t *act_codes, const uint8_t *act_scales,
                           const uint8_t *up, const uint16_t *up_s, const uint8_t *gate,
                           const uint16_t *gate_s, size_t m, size_t k, int layout, float *out);

/* ---- synthetic data generator (counter-based, identical spec in csrc/synth.hip) ---- */
uint64_t v3o_synth_hash(uint64_t seed, uint64_t stream, uint64_t ctr);
float v3o_synth_normal(uint64_t seed, uint64_t stream, uint64_t ctr);
/* n bytes of uniform bits: byte j = (hash(seed, stream, j/8) >> 8*(j%8)) & 0xff */
void v3o_synth_bytes(uint64_t seed, uint64_t stream, size_t off, size_t n, uint8_t *dst);
/* rounded |N(0,1)|*sigma in dt (bf16/f16), redrawn while it rounds to zero */
uint16_t v3o_synth_scale(uint64_t seed, uint64_t stream, uint64_t idx, float sigma, int dt);
/* normal(0,1)*sigma written as dt (f32/f16/bf16) for indices [off, off+n) */
void v3o_synth_normal_array(uint64_t seed, uint64_t stream, size_t off, size_t n, float sigma,
                            int dt, void *dst);
/* Write rows [row_start, row_start+rows) of the logical INT4 matrix (stream, k, g) as one page. */
void v3o_synth_int4_page(uint64_t seed, uint64_t stream, size_t k, size_t g, int scale_dt,
                         float sigma, size_t row_start, size_t rows, uint8_t *page);

/* E8M0 scale byte 119 + hash % 5 (2^-8 .. 2^-4) and an MXFP4 page of the logical matrix
 * `stream`: codes from stream*2 (uniform over all 16), scales from stream*2+1. */
uint8_t v3o_synth_e8m0(uint64_t seed, uint64_t stream, uint64_t idx);
void v3o_synth_mxfp4_page(uint64_t seed, uint64_t stream, size_t k, size_t row_start, size_t rows,
                          uint8_t *page);

#ifdef __cplusplus
}
#endif
#endif
