/*
 * oracle/cpu_ref.c — CPU restatement of vib3's MoE expert path. TEST INFRASTRUCTURE ONLY:
 * the HIP product never links or calls this file; tests/ and bench.py's cpu_baseline leg do.
 *
 * Built with -O2 -ffp-contract=off (see oracle/Makefile) so that every `acc += a * b` is a
 * rounded multiply followed by a rounded add, exactly as rustc compiles the reference loops
 * (Rust never contracts a*b+c into an FMA). Row parallelism (rayon in the reference,
 * kernels.rs:2658 PARALLEL_ROW_THRESHOLD = 64) only changes which thread computes a row,
 * never the arithmetic, so pthreads over row ranges reproduce it.
 */
#include "cpu_ref.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>
#include <unistd.h>

/* ------------------------------------------------------------------ conversions */

static inline uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

/* f32 -> f16, round to nearest even, subnormals and overflow to inf, NaN kept quiet. */
uint16_t v3o_f32_to_f16(float f)
{
    uint32_t x = f2u(f);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t exp = (x >> 23) & 0xffu;
    uint32_t man = x & 0x7fffffu;
    if (exp == 0xff) {
        if (man == 0) return (uint16_t)(sign | 0x7c00u);
        return (uint16_t)(sign | 0x7e00u | (man >> 13));
    }
    int e = (int)exp - 127 + 15;
    if (e >= 0x1f) return (uint16_t)(sign | 0x7c00u);
    if (e <= 0) {
        /* subnormal half: value = man24 * 2^(exp-150); half quantum 2^-24 */
        if (e < -10) return (uint16_t)sign; /* below half of the smallest subnormal */
        uint32_t m = man | 0x800000u;       /* 24-bit significand */
        uint32_t shift = (uint32_t)(14 - e); /* bits to drop: 13 + (1 - e) */
        uint32_t half_m = m >> shift;
        uint32_t rem = m & ((1u << shift) - 1u);
        uint32_t halfway = 1u << (shift - 1u);
        if (rem > halfway || (rem == halfway && (half_m & 1u))) half_m++;
        return (uint16_t)(sign | half_m);
    }
    uint32_t half_m = man >> 13;
    uint32_t rem = man & 0x1fffu;
    uint32_t out = sign | ((uint32_t)e << 10) | half_m;
    if (rem > 0x1000u || (rem == 0x1000u && (half_m & 1u))) out++; /* carries into exp ok */
    return (uint16_t)out;
}

float v3o_f16_to_f32(uint16_t h)
{
    uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
    uint32_t exp = (h >> 10) & 0x1fu;
    uint32_t man = h & 0x3ffu;
    if (exp == 0) {
        if (man == 0) return u2f(sign);
        /* subnormal: man * 2^-24 exactly */
        float v = (float)man * 5.9604644775390625e-08f;
        return sign ? -v : v;
    }
    if (exp == 0x1f) return u2f(sign | 0x7f800000u | (man << 13));
    return u2f(sign | ((exp + 112u) << 23) | (man << 13));
}

/* half::bf16::from_f32: NaN -> quiet NaN of the top bits, otherwise round to nearest even. */
uint16_t v3o_f32_to_bf16(float f)
{
    uint32_t x = f2u(f);
    if ((x & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((x >> 16) | 0x0040u);
    uint32_t round_bit = 0x8000u;
    if ((x & round_bit) != 0 && (x & (3u * round_bit - 1u)) != 0) return (uint16_t)((x >> 16) + 1u);
    return (uint16_t)(x >> 16);
}

float v3o_bf16_to_f32(uint16_t b) { return u2f((uint32_t)b << 16); }

void v3o_to_f32(const void *src, int dt, size_t n, float *dst)
{
    if (dt == V3O_F32) { memcpy(dst, src, n * 4); return; }
    const uint16_t *s = (const uint16_t *)src;
    for (size_t i = 0; i < n; i++)
        dst[i] = dt == V3O_F16 ? v3o_f16_to_f32(s[i]) : v3o_bf16_to_f32(s[i]);
}

static inline float decode_scale(const uint8_t *p, int dt)
{
    uint16_t bits = (uint16_t)(p[0] | (p[1] << 8));
    return dt == V3O_F16 ? v3o_f16_to_f32(bits) : v3o_bf16_to_f32(bits);
}

/* kernels.rs:2789-2797: a scale that is not finite or not > 0 decodes as 1/8. */
static inline float valid_scale(float s) { return (isfinite(s) && s > 0.0f) ? s : 0.125f; }

/* ------------------------------------------------------------------ threading */

int v3o_default_threads(void)
{
    const char *env = getenv("VIB3_ORACLE_THREADS");
    if (env && atoi(env) > 0) return atoi(env);
    long n = sysconf(_SC_NPROCESSORS_ONLN);
    return n > 0 ? (int)n : 1;
}

typedef void (*row_fn)(void *ctx, size_t r0, size_t r1);
typedef struct { row_fn fn; void *ctx; size_t r0, r1; } row_job;

static void *row_thread(void *p)
{
    row_job *j = (row_job *)p;
    j->fn(j->ctx, j->r0, j->r1);
    return NULL;
}

/* Run fn over [0, m) split into contiguous ranges; sequential below 64 rows like the
 * reference (kernels.rs:2658). */
static void parallel_rows(size_t m, int nthreads, row_fn fn, void *ctx)
{
    if (nthreads <= 0) nthreads = v3o_default_threads();
    if (m < 64 || nthreads == 1) { fn(ctx, 0, m); return; }
    if ((size_t)nthreads > m) nthreads = (int)m;
    pthread_t *th = (pthread_t *)malloc(sizeof(pthread_t) * (size_t)nthreads);
    row_job *jobs = (row_job *)malloc(sizeof(row_job) * (size_t)nthreads);
    size_t per = (m + (size_t)nthreads - 1) / (size_t)nthreads;
    int started = 0;
    for (int t = 0; t < nthreads; t++) {
        size_t r0 = (size_t)t * per, r1 = r0 + per > m ? m : r0 + per;
        if (r0 >= r1) break;
        jobs[t] = (row_job){fn, ctx, r0, r1};
        if (pthread_create(&th[t], NULL, row_thread, &jobs[t]) != 0) { fn(ctx, r0, r1); continue; }
        started = t + 1;
    }
    for (int t = 0; t < started; t++) pthread_join(th[t], NULL);
    free(th);
    free(jobs);
}

/* ------------------------------------------------------------------ INT4 GEMV */

typedef struct {
    const float *x;
    const uint8_t *page;
    size_t k, m, g;
    int sdt;
    float *acc;
} int4_ctx;

/* One row of cpu_matmul_int4_grouped (kernels.rs:2770-2820): build the 16-entry LUT per group,
 * then the byte loop: acc += x[col] * lut[lo]; acc += x[col+1] * lut[hi]. */
static float int4_row(const float *x, const uint8_t *page, size_t k, size_t m, size_t g, int sdt,
                      size_t row, float *lut /* [G*16] */)
{
    size_t pk = (k + 1) / 2, ng = (k + g - 1) / g;
    const uint8_t *rowp = page + row * pk;
    const uint8_t *sc = page + pk * m + row * ng * 2;
    for (size_t gi = 0; gi < ng; gi++) {
        float s = valid_scale(decode_scale(sc + gi * 2, sdt));
        for (int q = 0; q < 16; q++) lut[gi * 16 + (size_t)q] = (float)(q - 8) * s;
    }
    float acc = 0.0f;
    for (size_t b = 0; b < pk; b++) {
        size_t col = b * 2;
        if (col >= k) break;
        size_t gi = col / g;
        if (gi > ng - 1) gi = ng - 1;
        uint8_t p = rowp[b];
        acc += x[col] * lut[gi * 16 + (p & 0x0f)];
        if (col + 1 < k) acc += x[col + 1] * lut[gi * 16 + (p >> 4)];
    }
    return acc;
}

static void int4_rows(void *vctx, size_t r0, size_t r1)
{
    int4_ctx *c = (int4_ctx *)vctx;
    size_t ng = (c->k + c->g - 1) / c->g;
    float *lut = (float *)malloc(sizeof(float) * 16 * ng);
    for (size_t r = r0; r < r1; r++) c->acc[r] = int4_row(c->x, c->page, c->k, c->m, c->g, c->sdt, r, lut);
    free(lut);
}

void v3o_matmul_int4_acc(const float *x, const uint8_t *page, size_t k, size_t m, size_t g,
                         int scale_dt, float *acc, int nthreads)
{
    int4_ctx c = {x, page, k, m, g, scale_dt, acc};
    parallel_rows(m, nthreads, int4_rows, &c);
}

void v3o_partial_matmul_int4(const uint16_t *x_f16, const uint8_t *page, uint16_t *out_f16,
                             size_t k, size_t m)
{
    float *x = (float *)malloc(sizeof(float) * k);
    float *acc = (float *)malloc(sizeof(float) * m);
    for (size_t i = 0; i < k; i++) x[i] = v3o_f16_to_f32(x_f16[i]);
    v3o_matmul_int4_acc(x, page, k, m, 32, V3O_BF16, acc, 0);
    for (size_t r = 0; r < m; r++) out_f16[r] = v3o_f32_to_f16(acc[r]);
    free(x);
    free(acc);
}

/* ------------------------------------------------------------------ INT4 SwiGLU */

typedef struct {
    const float *x;
    const uint8_t *up, *gate;
    size_t k, m, g;
    int sdt;
    float *h;
} swiglu_ctx;

static inline float silu_times(float gate, float up)
{
    /* kernels.rs:3041: silu = gate / (1 + (-gate).exp()); silu * up */
    float silu = gate / (1.0f + expf(-gate));
    return silu * up;
}

/* cpu_swiglu_int4 (kernels.rs:2959-3043): the two dot products interleave per byte, but each
 * accumulator sees exactly the same sequence of rounded operations as a single-matrix row. */
static void swiglu_rows(void *vctx, size_t r0, size_t r1)
{
    swiglu_ctx *c = (swiglu_ctx *)vctx;
    size_t ng = (c->k + c->g - 1) / c->g;
    float *lut = (float *)malloc(sizeof(float) * 16 * ng);
    for (size_t r = r0; r < r1; r++) {
        float up = int4_row(c->x, c->up, c->k, c->m, c->g, c->sdt, r, lut);
        float gate = int4_row(c->x, c->gate, c->k, c->m, c->g, c->sdt, r, lut);
        c->h[r] = silu_times(gate, up);
    }
    free(lut);
}

void v3o_swiglu_int4_acc(const float *x, const uint8_t *up_page, const uint8_t *gate_page,
                         size_t k, size_t m, size_t g, int scale_dt, float *h, int nthreads)
{
    swiglu_ctx c = {x, up_page, gate_page, k, m, g, scale_dt, h};
    parallel_rows(m, nthreads, swiglu_rows, &c);
}

void v3o_partial_swiglu_int4(const uint16_t *x_f16, const uint8_t *up_page,
                             const uint8_t *gate_page, uint16_t *out_f16, size_t k, size_t m)
{
    float *x = (float *)malloc(sizeof(float) * k);
    float *h = (float *)malloc(sizeof(float) * m);
    for (size_t i = 0; i < k; i++) x[i] = v3o_f16_to_f32(x_f16[i]);
    v3o_swiglu_int4_acc(x, up_page, gate_page, k, m, 32, V3O_BF16, h, 0);
    for (size_t r = 0; r < m; r++) out_f16[r] = v3o_f32_to_f16(h[r]);
    free(x);
    free(h);
}

/* ------------------------------------------------------------------ accumulate */

void v3o_weighted_accumulate_f32(float *out, const uint16_t *expert_f16, float w, size_t n)
{
    for (size_t i = 0; i < n; i++) out[i] += w * v3o_f16_to_f32(expert_f16[i]);
}

/* kernels.rs:1959-1996 weighted_accumulate CPU branch: f16 accumulator,
 * o = f16(f32(o) + w * f32(e)). */
void v3o_weighted_accumulate_f16(uint16_t *out, const uint16_t *expert_f16, float w, size_t n)
{
    for (size_t i = 0; i < n; i++)
        out[i] = v3o_f32_to_f16(v3o_f16_to_f32(out[i]) + w * v3o_f16_to_f32(expert_f16[i]));
}

/* ------------------------------------------------------------------ router */

typedef struct {
    const float *x;
    const void *w;
    int wdt;
    size_t d;
    float *scores;
} router_ctx;

static void router_rows(void *vctx, size_t r0, size_t r1)
{
    router_ctx *c = (router_ctx *)vctx;
    for (size_t e = r0; e < r1; e++) {
        float acc = 0.0f;
        if (c->wdt == V3O_F32) {
            const float *row = (const float *)c->w + e * c->d;
            for (size_t i = 0; i < c->d; i++) acc += c->x[i] * row[i];
        } else {
            const uint16_t *row = (const uint16_t *)c->w + e * c->d;
            for (size_t i = 0; i < c->d; i++)
                acc += c->x[i] * (c->wdt == V3O_F16 ? v3o_f16_to_f32(row[i]) : v3o_bf16_to_f32(row[i]));
        }
        c->scores[e] = acc;
    }
}

/* Stable descending selection of the k largest keys: equal keys keep ascending index order,
 * which is what Rust's stable `sort_by(|a, b| b.partial_cmp(a))` + truncate(k) yields for
 * non-NaN keys (kernels.rs:2370-2371, :2416-2417). */
static void stable_topk_desc(const float *key, size_t n, size_t k, size_t *idx_out)
{
    unsigned char *taken = (unsigned char *)calloc(n, 1);
    for (size_t j = 0; j < k; j++) {
        size_t best = (size_t)-1;
        for (size_t i = 0; i < n; i++) {
            if (taken[i]) continue;
            if (best == (size_t)-1 || key[i] > key[best]) best = i;
        }
        taken[best] = 1;
        idx_out[j] = best;
    }
    free(taken);
}

int v3o_router(const float *x, const void *w, int w_dt, size_t num_experts, size_t hidden,
               size_t top_k, int mode, float scaling, int normalize, const float *bias,
               uint16_t *ids, float *weights, float *scores_out, int nthreads)
{
    if (top_k == 0 || top_k > num_experts || num_experts > 65536) return -1;
    float *scores = (float *)malloc(sizeof(float) * num_experts);
    router_ctx c = {x, w, w_dt, hidden, scores};
    parallel_rows(num_experts, nthreads, router_rows, &c);
    if (scores_out) memcpy(scores_out, scores, sizeof(float) * num_experts);
    size_t *sel = (size_t *)malloc(sizeof(size_t) * top_k);
    if (mode == 0) {
        /* kernels.rs:2368-2387 */
        stable_topk_desc(scores, num_experts, top_k, sel);
        float mx = -INFINITY;
        for (size_t j = 0; j < top_k; j++) mx = fmaxf(mx, scores[sel[j]]);
        float sum = 0.0f;
        for (size_t j = 0; j < top_k; j++) sum += expf(scores[sel[j]] - mx);
        for (size_t j = 0; j < top_k; j++) {
            ids[j] = (uint16_t)sel[j];
            weights[j] = expf(scores[sel[j]] - mx) / sum;
        }
    } else {
        /* kernels.rs:2389-2436 */
        float *sig = (float *)malloc(sizeof(float) * num_experts);
        float *selk = (float *)malloc(sizeof(float) * num_experts);
        for (size_t e = 0; e < num_experts; e++) {
            sig[e] = 1.0f / (1.0f + expf(-scores[e]));
            selk[e] = bias ? sig[e] + bias[e] : sig[e];
        }
        stable_topk_desc(selk, num_experts, top_k, sel);
        for (size_t j = 0; j < top_k; j++) { ids[j] = (uint16_t)sel[j]; weights[j] = sig[sel[j]]; }
        if (normalize) {
            float total = 0.0f;
            for (size_t j = 0; j < top_k; j++) total += weights[j];
            if (total > 1e-20f)
                for (size_t j = 0; j < top_k; j++) weights[j] /= total;
        }
        for (size_t j = 0; j < top_k; j++) weights[j] *= scaling;
        free(sig);
        free(selk);
    }
    free(sel);
    free(scores);
    return 0;
}

/* ------------------------------------------------------------------ quantizer */

/* quantize_weights_to_int4 (kernels.rs:3778-3831) with g as a parameter. Rust's f32::round is
 * half-away-from-zero, which is C's roundf; `as i32` then clamp(0, 15). */
void v3o_quantize_int4(const float *w, size_t rows, size_t cols, size_t g, uint8_t *out)
{
    size_t pk = (cols + 1) / 2, ng = (cols + g - 1) / g;
    memset(out, 0, rows * pk + rows * ng * 2);
    uint8_t *sc = out + rows * pk;
    for (size_t r = 0; r < rows; r++) {
        const float *row = w + r * cols;
        for (size_t gi = 0; gi < ng; gi++) {
            size_t c0 = gi * g, c1 = c0 + g < cols ? c0 + g : cols;
            float mx = 0.0f;
            for (size_t c = c0; c < c1; c++) mx = fmaxf(mx, fabsf(row[c]));
            float scale = mx > 0.0f ? mx / 7.0f : 1.0f;
            uint16_t sb = v3o_f32_to_bf16(scale);
            sc[(r * ng + gi) * 2] = (uint8_t)(sb & 0xff);
            sc[(r * ng + gi) * 2 + 1] = (uint8_t)(sb >> 8);
            for (size_t c = c0; c < c1; c++) {
                int q = (int)roundf(row[c] / scale) + 8;
                q = q < 0 ? 0 : (q > 15 ? 15 : q);
                if (c % 2 == 0) out[r * pk + c / 2] |= (uint8_t)(q & 0x0f);
                else out[r * pk + c / 2] |= (uint8_t)((q & 0x0f) << 4);
            }
        }
    }
}

/* dequantize_int4_to_f32 (kernels.rs:3866-3927): (q - 8) * scale, scale in dt. */
void v3o_dequantize_int4(const uint8_t *page, size_t rows, size_t cols, size_t g, int scale_dt,
                         float *out)
{
    size_t pk = (cols + 1) / 2, ng = (cols + g - 1) / g;
    const uint8_t *sc = page + rows * pk;
    for (size_t r = 0; r < rows; r++)
        for (size_t c = 0; c < cols; c++) {
            uint8_t b = page[r * pk + c / 2];
            int q = (c % 2 == 0) ? (b & 0x0f) : (b >> 4);
            float s = decode_scale(sc + (r * ng + c / g) * 2, scale_dt);
            out[r * cols + c] = (float)(q - 8) * s;
        }
}

/* ------------------------------------------------------------------ MoE layer */

/* execute_expert (engine.rs:5801-6306) for INT4 pages: up/gate pages are paired in order and
 * each pair writes rows [p*R, p*R + rows) of h; each down page reads the whole h. */
static void run_expert(const float *x, size_t hidden, size_t inter, size_t g, int sdt,
                       const v3o_expert *ex, float weight, int faithful, float *out, int nthreads)
{
    float *h = (float *)calloc(inter, sizeof(float));
    float *tmp = (float *)malloc(sizeof(float) * (inter > hidden ? inter : hidden));
    for (size_t p = 0; p < ex->up.npages && p < ex->gate.npages; p++) {
        size_t r0 = p * ex->up.rows_per_page;
        size_t rows = inter - r0 < ex->up.rows_per_page ? inter - r0 : ex->up.rows_per_page;
        v3o_swiglu_int4_acc(x, ex->up.pages[p], ex->gate.pages[p], hidden, rows, g, sdt, tmp,
                            nthreads);
        for (size_t r = 0; r < rows; r++)
            h[r0 + r] = faithful ? v3o_f16_to_f32(v3o_f32_to_f16(tmp[r])) : tmp[r];
    }
    for (size_t p = 0; p < ex->down.npages; p++) {
        size_t r0 = p * ex->down.rows_per_page;
        size_t rows = hidden - r0 < ex->down.rows_per_page ? hidden - r0 : ex->down.rows_per_page;
        v3o_matmul_int4_acc(h, ex->down.pages[p], inter, rows, g, sdt, tmp, nthreads);
        for (size_t r = 0; r < rows; r++) {
            float d = faithful ? v3o_f16_to_f32(v3o_f32_to_f16(tmp[r])) : tmp[r];
            out[r0 + r] += weight * d; /* weighted_accumulate_f32, kernels.rs:2033 */
        }
    }
    free(h);
    free(tmp);
}

void v3o_moe_layer_w(const float *x, size_t hidden, size_t inter, size_t g, int scale_dt,
                     const v3o_expert *routed, const uint16_t *ids, const float *weights,
                     size_t top_k, const v3o_expert *shared, size_t n_shared,
                     const float *shared_w, int faithful, float *out, int nthreads)
{
    memset(out, 0, sizeof(float) * hidden); /* layer_output_buf.zero_async, engine.rs:5200 */
    for (size_t j = 0; j < top_k; j++)
        run_expert(x, hidden, inter, g, scale_dt, &routed[ids[j]], weights[j], faithful, out, nthreads);
    /* shared experts: weight 1.0 (weighted_accumulate_f32, engine.rs:6441-6449) or the sigmoid
     * of the gate (sigmoid_gated_accumulate_f32, engine.rs:6418-6424) */
    for (size_t s = 0; s < n_shared; s++)
        run_expert(x, hidden, inter, g, scale_dt, &shared[s], shared_w ? shared_w[s] : 1.0f,
                   faithful, out, nthreads);
}

void v3o_moe_layer(const float *x, size_t hidden, size_t inter, size_t g, int scale_dt,
                   const v3o_expert *routed, const uint16_t *ids, const float *weights,
                   size_t top_k, const v3o_expert *shared, size_t n_shared, int faithful,
                   float *out, int nthreads)
{
    v3o_moe_layer_w(x, hidden, inter, g, scale_dt, routed, ids, weights, top_k, shared, n_shared,
                    NULL, faithful, out, nthreads);
}

/* ------------------------------------------------------------------ either side of the MoE */

/* vib3_rms_norm_f32 (kernels.cu:921-955): 256 strided partial sums of squares (the CUDA
 * compiler contracts `partial_ss += val * val` into a fused multiply-add), a halving tree over
 * the 256 partials, rms = sqrtf(ss / n + eps), inv = 1 / rms, y = (x * inv) * w. */
float v3o_inv_rms(const float *x, size_t n, float eps)
{
    float part[256];
    for (size_t t = 0; t < 256; t++) {
        float p = 0.0f;
        for (size_t d = t; d < n; d += 256) p = fmaf(x[d], x[d], p);
        part[t] = p;
    }
    for (size_t s = 128; s > 0; s >>= 1)
        for (size_t t = 0; t < s; t++) part[t] = part[t] + part[t + s];
    float rms = sqrtf(part[0] / (float)n + eps);
    return 1.0f / rms;
}

void v3o_rms_norm_f32(const float *x, size_t n, const uint16_t *w_f16, float eps, float *out)
{
    float inv = v3o_inv_rms(x, n, eps);
    for (size_t d = 0; d < n; d++) out[d] = x[d] * inv * v3o_f16_to_f32(w_f16[d]);
}

/* vib3_residual_add_f32_f32_kernel (kernels.cu:817): acc[i] += lo[i]. */
void v3o_residual_add_f32(float *acc, const float *lo, size_t n)
{
    for (size_t i = 0; i < n; i++) acc[i] = acc[i] + lo[i];
}

/* linear_projection_f32_to_f32 CPU body (kernels.rs:3630-3640): one output row, sequential
 * acc += x[d] * f32(w[d]); used for the shared expert's gate logit (engine.rs:6396). */
float v3o_linear_row_f16(const float *x, const uint16_t *w_f16, size_t n)
{
    float acc = 0.0f;
    for (size_t d = 0; d < n; d++) acc += x[d] * v3o_f16_to_f32(w_f16[d]);
    return acc;
}

/* the gate's sigmoid (kernels.cu:2114): 1 / (1 + exp(-g)) */
float v3o_sigmoid(float g) { return 1.0f / (1.0f + expf(-g)); }

/* ------------------------------------------------------------------ MXFP4 */

/* kernels.cu:438-441: bit3 sign, bits2-1 exponent, bit0 mantissa. */
float v3o_e2m1(uint8_t code)
{
    static const float mag[8] = {0.0f, 0.5f, 1.0f, 1.5f, 2.0f, 3.0f, 4.0f, 6.0f};
    float v = mag[code & 7];
    return (code & 8) ? -v : v;
}

/* kernels.cu:2770-2777: the E8M0 byte is placed in the f32 exponent field: 2^(e-127), e=0 -> 0. */
float v3o_e8m0(uint8_t e) { return u2f((uint32_t)e << 23); }

typedef struct {
    const float *x;
    const uint8_t *codes, *scales;
    size_t k, m;
    float *acc;
} mx_ctx;

static void mx_rows(void *vctx, size_t r0, size_t r1)
{
    mx_ctx *c = (mx_ctx *)vctx;
    size_t pk = (c->k + 1) / 2, nb = (c->k + 31) / 32;
    for (size_t r = r0; r < r1; r++) {
        float acc = 0.0f;
        for (size_t col = 0; col < c->k; col++) {
            uint8_t b = c->codes[r * pk + col / 2];
            uint8_t q = (col % 2 == 0) ? (b & 0x0f) : (b >> 4);
            float wv = v3o_e2m1(q) * v3o_e8m0(c->scales[r * nb + col / 32]);
            acc += c->x[col] * wv;
        }
        c->acc[r] = acc;
    }
}

void v3o_matmul_mxfp4_acc(const float *x, const uint8_t *codes, const uint8_t *scales, size_t k,
                          size_t m, float *acc, int nthreads)
{
    mx_ctx c = {x, codes, scales, k, m, acc};
    parallel_rows(m, nthreads, mx_rows, &c);
}

/* Batched MoE over MXFP4 experts, restated per token the way the engine decodes (there is no
 * multi-token MoE in the reference): per token, each pick runs execute_expert's composition
 * (engine.rs:5801-6306) with MXFP4 matrices, f16 rounding of h and d (kernels.rs:3042, :2825),
 * then weighted_accumulate_f32 in pick order (kernels.rs:2033); out is rounded to bf16. */
void v3o_moe_mxfp4_batched(const float *x, size_t tokens, size_t hidden, size_t inter,
                           const uint8_t *const *pages, size_t num_experts, const uint16_t *ids,
                           const float *weights, size_t top_k, uint16_t *out, int nthreads)
{
    float *gate = (float *)malloc(sizeof(float) * inter);
    float *up = (float *)malloc(sizeof(float) * inter);
    float *h = (float *)malloc(sizeof(float) * inter);
    float *d = (float *)malloc(sizeof(float) * hidden);
    float *o = (float *)malloc(sizeof(float) * hidden);
    for (size_t t = 0; t < tokens; t++) {
        const float *xt = x + t * hidden;
        memset(o, 0, sizeof(float) * hidden);
        for (size_t j = 0; j < top_k; j++) {
            size_t e = ids[t * top_k + j];
            if (e >= num_experts) continue;
            const uint8_t *pu = pages[e * 3 + 0], *pg = pages[e * 3 + 1], *pd = pages[e * 3 + 2];
            v3o_matmul_mxfp4_acc(xt, pu, pu + inter * (hidden / 2), hidden, inter, up, nthreads);
            v3o_matmul_mxfp4_acc(xt, pg, pg + inter * (hidden / 2), hidden, inter, gate, nthreads);
            for (size_t r = 0; r < inter; r++)
                h[r] = v3o_f16_to_f32(v3o_f32_to_f16(silu_times(gate[r], up[r])));
            v3o_matmul_mxfp4_acc(h, pd, pd + hidden * (inter / 2), inter, hidden, d, nthreads);
            float w = weights[t * top_k + j];
            for (size_t r = 0; r < hidden; r++)
                o[r] += w * v3o_f16_to_f32(v3o_f32_to_f16(d[r]));
        }
        for (size_t r = 0; r < hidden; r++) out[t * hidden + r] = v3o_f32_to_bf16(o[r]);
    }
    free(gate);
    free(up);
    free(h);
    free(d);
    free(o);
}

/* ------------------------------------------------------------------ synthetic data */

static inline uint64_t mix64(uint64_t z)
{
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

uint64_t v3o_synth_hash(uint64_t seed, uint64_t stream, uint64_t ctr)
{
    uint64_t z = seed ^ (stream * 0xD1B54A32D192ED03ull);
    z += (ctr + 1ull) * 0x9E3779B97F4A7C15ull;
    z = mix64(z);
    return mix64(z + 0x9E3779B97F4A7C15ull);
}

/* Irwin-Hall(4) of 16-bit uniforms, centred and scaled to unit variance:
 * (sum - 131070) / 37837.23 with the constant rounded to f32 (2.6429e-5f). Integer sum is
 * exact; the single f32 multiply is the only rounding, so host and device agree bit for bit. */
float v3o_synth_normal(uint64_t seed, uint64_t stream, uint64_t ctr)
{
    uint64_t h = v3o_synth_hash(seed, stream, ctr);
    int32_t s = (int32_t)(h & 0xffff) + (int32_t)((h >> 16) & 0xffff) +
                (int32_t)((h >> 32) & 0xffff) + (int32_t)(h >> 48) - 131070;
    return (float)s * 2.6429e-5f;
}

void v3o_synth_bytes(uint64_t seed, uint64_t stream, size_t off, size_t n, uint8_t *dst)
{
    for (size_t i = 0; i < n; i++) {
        size_t j = off + i;
        dst[i] = (uint8_t)(v3o_synth_hash(seed, stream, j >> 3) >> (8 * (j & 7)));
    }
}

static uint16_t round_to(float v, int dt)
{
    return dt == V3O_F16 ? v3o_f32_to_f16(v) : v3o_f32_to_bf16(v);
}

uint16_t v3o_synth_scale(uint64_t seed, uint64_t stream, uint64_t idx, float sigma, int dt)
{
    for (uint64_t t = 0;; t++) {
        float v = fabsf(v3o_synth_normal(seed, stream, idx + (t << 40))) * sigma;
        uint16_t b = round_to(v, dt);
        if ((b & 0x7fff) != 0) return b;
    }
}

void v3o_synth_normal_array(uint64_t seed, uint64_t stream, size_t off, size_t n, float sigma,
                            int dt, void *dst)
{
    for (size_t i = 0; i < n; i++) {
        float v = v3o_synth_normal(seed, stream, off + i) * sigma;
        if (dt == V3O_F32) ((float *)dst)[i] = v;
        else ((uint16_t *)dst)[i] = round_to(v, dt);
    }
}

void v3o_synth_int4_page(uint64_t seed, uint64_t stream, size_t k, size_t g, int scale_dt,
                         float sigma, size_t row_start, size_t rows, uint8_t *page)
{
    size_t pk = (k + 1) / 2, ng = (k + g - 1) / g;
    v3o_synth_bytes(seed, stream * 2, row_start * pk, rows * pk, page);
    uint8_t *sc = page + rows * pk;
    for (size_t i = 0; i < rows * ng; i++) {
        uint16_t b = v3o_synth_scale(seed, stream * 2 + 1, row_start * ng + i, sigma, scale_dt);
        sc[2 * i] = (uint8_t)(b & 0xff);
        sc[2 * i + 1] = (uint8_t)(b >> 8);
    }
}

/* E8M0 bytes 119 + hash % 5 (2^-8 .. 2^-4), as csrc/synth.hip's k_synth_e8m0. */
uint8_t v3o_synth_e8m0(uint64_t seed, uint64_t stream, uint64_t idx)
{
    return (uint8_t)(119 + v3o_synth_hash(seed, stream, idx) % 5);
}

void v3o_synth_mxfp4_page(uint64_t seed, uint64_t stream, size_t k, size_t row_start, size_t rows,
                          uint8_t *page)
{
    size_t pk = k / 2, nb = k / 32;
    v3o_synth_bytes(seed, stream * 2, row_start * pk, rows * pk, page);
    uint8_t *sc = page + rows * pk;
    for (size_t i = 0; i < rows * nb; i++)
        sc[i] = v3o_synth_e8m0(seed, stream * 2 + 1, row_start * nb + i);
}

/* ------------------------------------------------------------------ NVFP4 fused MoE
 * The reference's sync-free fused path (cuda/src/kernels.cu:5357-5591 kernels, :5650 / :5868
 * launchers) over split-half E2M1 data with block scales, restated element by element. */

/* kernels.cu:2759-2768 compute_e8m0: round(log2(amax)) - 2 + 127, clamped to [0, 254];
 * round(log2) evaluated exactly as floor(log2) + (mantissa > sqrt 2). */
uint8_t v3o_fp4_e8m0_of_amax(float amax)
{
    if (!(amax > 0.0f)) return 0;
    uint32_t b = f2u(amax);
    int E = (int)(b >> 23);
    if (E == 0) return 0;
    int n = E - 127 + ((b & 0x7fffff) > 0x3504f3 ? 1 : 0);
    int biased = n + 125;
    return (uint8_t)(biased < 0 ? 0 : biased > 254 ? 254 : biased);
}

/* E2M1 code of v: round to nearest on {0, .5, 1, 1.5, 2, 3, 4, 6}, ties to the even code,
 * saturating at 6, sign bit from v (cvt.rn.satfinite of __nv_fp4x4_e2m1, kernels.cu:3227). */
uint8_t v3o_e2m1_rne(float v)
{
    uint8_t sign = (uint8_t)((f2u(v) >> 31) << 3);
    float a = fabsf(v);
    uint8_t c;
    if (a <= 0.25f) c = 0;
    else if (a < 0.75f) c = 1;
    else if (a <= 1.25f) c = 2;
    else if (a < 1.75f) c = 3;
    else if (a <= 2.5f) c = 4;
    else if (a < 3.5f) c = 5;
    else if (a <= 5.0f) c = 6;
    else c = 7;
    return sign | c;
}

/* e^x: Cody-Waite reduction with a two-part ln2 and the degree-7 Taylor polynomial of e^r in
 * Horner form, then ldexp (the GPU kernel's exp, operation for operation). */
float v3o_exp_cw(float x)
{
    if (x != x) return x;
    if (x > 88.72283935546875f) return INFINITY;
    if (x < -103.97208404541015625f) return 0.0f;
    float n = rintf(x * 1.44269502162933349609375f);
    float r = x - n * 0.693145751953125f;
    r = r - n * 1.428606765330187045e-06f;
    float p = 1.0f / 5040.0f;
    p = p * r + 1.0f / 720.0f;
    p = p * r + 1.0f / 120.0f;
    p = p * r + 1.0f / 24.0f;
    p = p * r + 1.0f / 6.0f;
    p = p * r + 0.5f;
    p = p * r + 1.0f;
    p = p * r + 1.0f;
    return ldexpf(p, (int)n);
}

static float e8m0_inv(uint8_t e) { return e == 0 ? INFINITY : u2f((uint32_t)(254 - e) << 23); }

/* kernels.cu:3193-3240 vib3_quantize_activation_fp4_kernel: per 32 values, e = E8M0 of the
 * absolute maximum, inv = 1 / 2^(e-127) (0 when the group is all zero), code = E2M1(v * inv);
 * split-half: byte j of the group = code(v[j]) | code(v[j+16]) << 4. */
void v3o_fp4_quantize_act(const float *x, size_t k, uint8_t *codes, uint8_t *scales)
{
    size_t groups = (k + 31) / 32;
    for (size_t g = 0; g < groups; g++) {
        float v[32], amax = 0.0f;
        for (int i = 0; i < 32; i++) {
            v[i] = g * 32 + i < k ? x[g * 32 + i] : 0.0f;
            amax = fmaxf(amax, fabsf(v[i]));
        }
        uint8_t e = v3o_fp4_e8m0_of_amax(amax);
        float inv = amax == 0.0f ? 0.0f : e8m0_inv(e);
        for (int j = 0; j < 16; j++)
            if (g * 32 + j < k)
                codes[g * 16 + j] = (uint8_t)(v3o_e2m1_rne(v[j] * inv) |
                                              (v3o_e2m1_rne(v[j + 16] * inv) << 4));
        scales[g] = e;
    }
}

/* kernels.cu:6585-6702 vib3_fused_rms_norm_quantize_fp4_kernel (one 256-thread block):
 * thread t accumulates x[d]^2 for d = t, t + 256, ... (a fused multiply-add each, as the CUDA
 * compiler contracts `partial_ss += val * val`), each 32-thread warp sums its partials by the
 * butterfly xor 16, 8, 4, 2, 1, thread 0 adds the eight warp sums in order from 0; then
 * y[d] = (x[d] * inv) * f32(w[d]) (two rounded products), optionally rounded to f16, and y is
 * quantized as v3o_fp4_quantize_act. The reference takes inv = rsqrtf(ss / K + eps), CUDA's
 * approximate reciprocal square root; this restatement (and the GPU kernel) uses the
 * correctly rounded 1 / sqrtf(ss / K + eps). */
float v3o_fp4_norm_inv(const float *x, size_t k, float eps)
{
    float part[256];
    for (size_t t = 0; t < 256; t++) {
        float p = 0.0f;
        for (size_t d = t; d < k; d += 256) p = fmaf(x[d], x[d], p);
        part[t] = p;
    }
    float ws[8];
    for (int w = 0; w < 8; w++) {
        float v[32], nv[32];
        for (int l = 0; l < 32; l++) v[l] = part[w * 32 + l];
        for (int m = 16; m > 0; m >>= 1) {
            for (int l = 0; l < 32; l++) nv[l] = v[l] + v[l ^ m];
            for (int l = 0; l < 32; l++) v[l] = nv[l];
        }
        ws[w] = v[0];
    }
    float total = 0.0f;
    for (int w = 0; w < 8; w++) total += ws[w];
    return 1.0f / sqrtf(total / (float)k + eps);
}

void v3o_fused_rms_norm_quantize_fp4(const float *x, const uint16_t *w_f16, size_t k, float eps,
                                     uint8_t *codes, uint8_t *scales, uint16_t *f16_out)
{
    float inv = v3o_fp4_norm_inv(x, k, eps);
    float *y = (float *)malloc(k * sizeof(float));
    for (size_t d = 0; d < k; d++) {
        y[d] = x[d] * inv * v3o_f16_to_f32(w_f16[d]);
        if (f16_out) f16_out[d] = v3o_f32_to_f16(y[d]);
    }
    v3o_fp4_quantize_act(y, k, codes, scales);
    free(y);
}

/* Code of element k of a split-half vector (byte k/32*16 + k%16, high nibble for k%32 >= 16). */
static uint8_t split_code(const uint8_t *codes, size_t k)
{
    uint8_t b = codes[(k / 32) * 16 + (k % 16)];
    return (k % 32) < 16 ? (b & 15) : (b >> 4);
}

/* Code of W[row][k] in the tiled split-half layout (kernels.cu:4185-4197). */
static uint8_t tiled_code(const uint8_t *data, size_t row, size_t k, size_t K)
{
    size_t nkt = K / 64, t = k / 64, grp = (k % 64) / 32, j = k % 32;
    uint8_t b = data[((row / 16) * nkt + t) * 512 + (row % 16) * 32 + grp * 16 + (j % 16)];
    return j < 16 ? (b & 15) : (b >> 4);
}

/* out[r] = f32( sum_k e2m1(W[r][k]) 2^(ew(r,k/32)-127) * e2m1(a[k]) 2^(ea(k/32)-127) ), with
 * ew the exponent byte of the row's bf16 scale (scale >> 7 & 0xff, kernels.cu:5404-5411): the
 * exact value (f64, exact for scale spreads below 2^33) rounded once to f32. */
void v3o_nvfp4_matvec(const uint8_t *act_codes, const uint8_t *act_scales, const uint8_t *data,
                      const uint16_t *scales, size_t m, size_t k, float *out)
{
    size_t G = k / 32;
    for (size_t r = 0; r < m; r++) {
        double acc = 0.0;
        for (size_t g = 0; g < G; g++) {
            double s = 0.0;
            for (size_t j = 0; j < 32; j++) {
                size_t kk = g * 32 + j;
                s += (double)v3o_e2m1(tiled_code(data, r, kk, k)) *
                     (double)v3o_e2m1(split_code(act_codes, kk));
            }
            int ew = (scales[r * G + g] >> 7) & 0xff;
            acc += s * ldexp(1.0, ew + (int)act_scales[g] - 254);
        }
        out[r] = (float)acc;
    }
}

/* kernels.cu:5650 / :5868: for each active expert e (pages: up, gate, down tiled data and their
 * scale arrays): u = up.a, g = gate.a (f32), h = (g * sigmoid(g)) * u with sigmoid = 1 / (1 +
 * e^-g) (:5485-5487), h quantized like the activation (:5451-5517), d = down.h, then
 * out[r] = out[r] + w_e * d[r] in expert order. */
void v3o_moe_experts_fused(const uint8_t *act_codes, const uint8_t *act_scales,
                           const uint8_t *const *data, const uint16_t *const *scales,
                           const float *weights, size_t n, size_t k_in, size_t m_mid,
                           size_t m_out, float *out)
{
    float *u = (float *)malloc(sizeof(float) * m_mid);
    float *gt = (float *)malloc(sizeof(float) * m_mid);
    float *h = (float *)malloc(sizeof(float) * m_mid);
    uint8_t *hc = (uint8_t *)malloc(m_mid / 2 + 16);
    uint8_t *hs = (uint8_t *)malloc(m_mid / 32 + 1);
    float *d = (float *)malloc(sizeof(float) * m_out);
    for (size_t e = 0; e < n; e++) {
        v3o_nvfp4_matvec(act_codes, act_scales, data[e * 3 + 0], scales[e * 3 + 0], m_mid, k_in, u);
        v3o_nvfp4_matvec(act_codes, act_scales, data[e * 3 + 1], scales[e * 3 + 1], m_mid, k_in, gt);
        for (size_t i = 0; i < m_mid; i++) {
            float sig = 1.0f / (1.0f + v3o_exp_cw(-gt[i]));
            h[i] = (gt[i] * sig) * u[i];
        }
        v3o_fp4_quantize_act(h, m_mid, hc, hs);
        v3o_nvfp4_matvec(hc, hs, data[e * 3 + 2], scales[e * 3 + 2], m_out, m_mid, d);
        for (size_t r = 0; r < m_out; r++) out[r] = out[r] + weights[e] * d[r];
    }
    free(u); free(gt); free(h); free(hc); free(hs); free(d);
}

/* kernels.cu:4132-4160: sequential -> split-half per 16-byte block (a partial block is left). */
void v3o_fp4_split_half(uint8_t *data, size_t nbytes)
{
    for (size_t b = 0; b + 16 <= nbytes; b += 16) {
        uint8_t t[16];
        memcpy(t, data + b, 16);
        for (int j = 0; j < 8; j++) {
            data[b + 2 * j] = (uint8_t)((t[j] & 0x0f) | ((t[j + 8] & 0x0f) << 4));
            data[b + 2 * j + 1] = (uint8_t)((t[j] >> 4) | (t[j + 8] & 0xf0));
        }
    }
}

/* kernels.cu:4190-4225: row-major [m][k/2] -> tiles of 16 rows x 32 bytes. */
void v3o_fp4_to_tiled(const uint8_t *src, uint8_t *dst, size_t m, size_t k)
{
    size_t pk = k / 2, nkt = pk / 32;
    for (size_t row = 0; row < (m / 16) * 16; row++)
        for (size_t t = 0; t < nkt; t++)
            memcpy(dst + ((row / 16) * nkt + t) * 512 + (row % 16) * 32, src + row * pk + t * 32, 32);
}

/* ------------------------------------------------------------------ NVFP4 weight quantizers */

/* Nearest E2M1 magnitude index of a non-negative value by the midpoint ladder of
 * kernels.rs:3952-3970 / :4052-4072 (a value on a midpoint goes to the larger magnitude;
 * NaN compares false everywhere and lands on 7). */
static uint8_t nvfp4_nearest(float v)
{
    static const float mid[7] = {0.25f, 0.75f, 1.25f, 1.75f, 2.5f, 3.5f, 5.0f};
    for (uint8_t i = 0; i < 7; i++)
        if (v < mid[i]) return i;
    return 7;
}

/* One row of kernels.rs:4085-4170 (quantize_weights_to_nvfp4) and of the second half of
 * :3998-4040 (convert_int4_to_nvfp4): per block of 32 columns, scale = max|w| / 6 in f32
 * (1.0 for an all-zero block), stored as f16; nibble = nearest(min(|w| / scale, 6)) with the
 * sign in bit 3 for w < 0; even column in the low nibble. Rust's f32::max / f32::min ignore a
 * NaN operand, as fmaxf / fminf do. */
static void nvfp4_quant_row(const float *row, size_t cols, uint8_t *data, uint8_t *scales)
{
    const size_t nb = (cols + 31) / 32;
    for (size_t b = 0; b < nb; b++) {
        const size_t c0 = b * 32, c1 = c0 + 32 < cols ? c0 + 32 : cols;
        float amax = 0.0f;
        for (size_t c = c0; c < c1; c++) amax = fmaxf(amax, fabsf(row[c]));
        const float scale = amax > 0.0f ? amax / 6.0f : 1.0f;
        const uint16_t sb = v3o_f32_to_f16(scale);
        scales[2 * b] = (uint8_t)(sb & 0xff);
        scales[2 * b + 1] = (uint8_t)(sb >> 8);
        for (size_t c = c0; c < c1; c++) {
            const float v = row[c];
            const uint8_t sign = v < 0.0f ? 1 : 0;
            const uint8_t nib = (uint8_t)(nvfp4_nearest(fminf(fabsf(v) / scale, 6.0f)) | (sign << 3));
            data[c / 2] |= (uint8_t)((c % 2 == 0) ? (nib & 0x0f) : ((nib & 0x0f) << 4));
        }
    }
}

size_t v3o_nvfp4_page_bytes(size_t rows, size_t cols)
{
    return rows * ((cols + 1) / 2) + rows * ((cols + 31) / 32) * 2;
}

void v3o_quantize_weights_to_nvfp4(const float *w, size_t rows, size_t cols, uint8_t *out)
{
    const size_t pk = (cols + 1) / 2, nb = (cols + 31) / 32;
    memset(out, 0, v3o_nvfp4_page_bytes(rows, cols));
    for (size_t r = 0; r < rows; r++)
        nvfp4_quant_row(w + r * cols, cols, out + r * pk, out + rows * pk + r * nb * 2);
}

/* kernels.rs:4172-4188: f16 / bf16 weights widened to f32, then the quantizer above. */
void v3o_quantize_half_to_nvfp4(const uint16_t *w, int dt, size_t rows, size_t cols,
                                uint8_t *out)
{
    float *f = (float *)malloc(rows * cols * sizeof(float));
    if (!f) return;
    v3o_to_f32(w, dt, rows * cols, f);
    v3o_quantize_weights_to_nvfp4(f, rows, cols, out);
    free(f);
}

/* kernels.rs:3937-4060 convert_int4_to_nvfp4: each INT4 row dequantized with its BF16 group
 * scales (w = (q - 8) * s; a scale whose two bytes lie past `len` reads as 1.0, the
 * reference's bounds rule), then quantized to NVFP4 as above. `len` is the INT4 buffer's
 * byte length. */
void v3o_convert_int4_to_nvfp4(const uint8_t *int4, size_t len, size_t rows, size_t cols,
                               size_t g, uint8_t *out)
{
    const size_t pk = (cols + 1) / 2, ng = (cols + g - 1) / g, nb = (cols + 31) / 32;
    const size_t tot = rows * pk;
    float *row = (float *)malloc(cols * sizeof(float));
    if (!row) return;
    memset(out, 0, v3o_nvfp4_page_bytes(rows, cols));
    for (size_t r = 0; r < rows; r++) {
        for (size_t j = 0; j < pk; j++) {
            const uint8_t b = int4[r * pk + j];
            const size_t c0 = 2 * j, c1 = c0 + 1;
            const size_t o0 = tot + (r * ng + c0 / g) * 2;
            const float s0 = o0 + 1 < len ? v3o_bf16_to_f32((uint16_t)(int4[o0] | (int4[o0 + 1] << 8)))
                                          : 1.0f;
            row[c0] = ((float)(b & 0x0f) - 8.0f) * s0;
            if (c1 < cols) {
                const size_t o1 = tot + (r * ng + c1 / g) * 2;
                const float s1 = o1 + 1 < len
                                     ? v3o_bf16_to_f32((uint16_t)(int4[o1] | (int4[o1 + 1] << 8)))
                                     : 1.0f;
                row[c1] = ((float)((b >> 4) & 0x0f) - 8.0f) * s1;
            }
        }
        nvfp4_quant_row(row, cols, out + r * pk, out + rows * pk + r * nb * 2);
    }
    free(row);
}

/* kernels.cu:6017-6128 vib3_fp16_to_nvfp4_weight_kernel: each row's 32-value groups quantized
 * like the activation (E8M0 of the group's absolute maximum, codes E2M1 round-to-nearest-even
 * of v * 2^(127-e), split-half within the group), the scale stored as the bf16 e << 7. This
 * follows the kernel's sm_120 branch (__nv_fp4x4_e2m1, cvt.rn.satfinite); its software branch
 * for older GPUs uses the midpoint ladder instead, which differs only on exact ties. */
void v3o_fp16_to_nvfp4_weight(const uint16_t *w_f16, size_t m, size_t k, uint8_t *data,
                              uint16_t *scales)
{
    const size_t G = k / 32;
    float *row = (float *)malloc(k * sizeof(float));
    uint8_t *e = (uint8_t *)malloc(G + 1);
    if (!row || !e) { free(row); free(e); return; }
    for (size_t r = 0; r < m; r++) {
        v3o_to_f32(w_f16 + r * k, V3O_F16, k, row);
        v3o_fp4_quantize_act(row, G * 32, data + r * (k / 2), e);
        for (size_t g = 0; g < G; g++) scales[r * G + g] = (uint16_t)(e[g] << 7);
    }
    free(row);
    free(e);
}

/* Row-major sequential NVFP4 (two codes per byte, low nibble = even column) with full BF16
 * block scales: out[r] = sum_k x[k] * e2m1(q) * bf16(s) in f64 (the reference's scalar GPU
 * kernels, kernels.cu:446-505, :1957-2090, accumulate per thread and reduce per warp, an
 * order this restatement does not fix; tests compare within a tolerance). */
void v3o_nvfp4_seq_matvec_f64(const float *x, const uint8_t *data, const uint16_t *scales,
                              size_t m, size_t k, double *out)
{
    const size_t pk = (k + 1) / 2, nb = (k + 31) / 32;
    for (size_t r = 0; r < m; r++) {
        double acc = 0.0;
        for (size_t c = 0; c < k; c++) {
            const uint8_t b = data[r * pk + c / 2];
            const uint8_t q = (c % 2 == 0) ? (b & 0x0f) : (b >> 4);
            acc += (double)x[c] * (double)v3o_e2m1(q) * (double)v3o_bf16_to_f32(scales[r * nb + c / 32]);
        }
        out[r] = acc;
    }
}

/* ------------------------------------------------------------------ per-page NVFP4 GEMVs */

/* Code of W[row][k] in layout `lay`: 0 = row-major split-half (kernels.cu:3739-3750, after
 * vib3_launch_repack_weights_inplace), 1 = tiled split-half (kernels.cu:4265), 2 = row-major
 * sequential (low nibble = even column, the quantizer's layout, kernels.cu:3387). */
static uint8_t layout_code(const uint8_t *data, size_t row, size_t k, size_t K, int lay)
{
    if (lay == 1) return tiled_code(data, row, k, K);
    const uint8_t *r = data + row * (K / 2);
    if (lay == 0) return split_code(r, k);
    const uint8_t b = r[k / 2];
    return (k % 2 == 0) ? (b & 15) : (b >> 4);
}

/* The block-scaled GEMV of the reference's per-page MMA kernels (kernels.cu:3276-3385,
 * :3739-3750, :4265-4358, :4438-4540) with a pre-quantized activation: out[r] = f32(exact
 * sum over groups g of (sum_j W e2m1 * a e2m1) * s_w(r, g) * 2^(ea_g - 127)), where s_w is
 * 2^(((s >> 7) & 0xff) - 127) (full = 0: the E8M0 byte the MMA instruction takes) or the bf16
 * value s (full = 1: vib3_gemv_scalar_nvfp4_kernel, kernels.cu:4480). Exact in f64 for the
 * scale spreads of real weights; rounded to f32 once. */
void v3o_nvfp4_page_matvec(const uint8_t *act_codes, const uint8_t *act_scales,
                           const uint8_t *data, const uint16_t *scales, size_t m, size_t k,
                           int layout, int full, float *out)
{
    const size_t G = k / 32;
    for (size_t r = 0; r < m; r++) {
        double acc = 0.0;
        for (size_t g = 0; g < G; g++) {
            double s = 0.0;
            for (size_t j = 0; j < 32; j++) {
                const size_t kk = g * 32 + j;
                s += (double)v3o_e2m1(layout_code(data, r, kk, k, layout)) *
                     (double)v3o_e2m1(split_code(act_codes, kk));
            }
            const uint16_t sw = scales[r * G + g];
            const double ws = full ? (double)v3o_bf16_to_f32(sw) : ldexp(1.0, ((sw >> 7) & 0xff) - 127);
            acc += s * ws * ldexp(1.0, (int)act_scales[g] - 127);
        }
        out[r] = (float)acc;
    }
}

/* SwiGLU of two page GEMVs as the reference composes it (kernels.cu:3853-3905 then
 * vib3_swiglu_fuse_f32_kernel :3789-3800): h = (g * sigmoid(g)) * u, sigmoid = 1 / (1 + e^-g)
 * with this file's exp (v3o_exp_cw). */
void v3o_nvfp4_page_swiglu(const uint8_t *act_codes, const uint8_t *act_scales,
                           const uint8_t *up, const uint16_t *up_s, const uint8_t *gate,
                           const uint16_t *gate_s, size_t m, size_t k, int layout, float *out)
{
    float *u = (float *)malloc(m * sizeof(float)), *g = (float *)malloc(m * sizeof(float));
    if (!u || !g) { free(u); free(g); return; }
    v3o_nvfp4_page_matvec(act_codes, act_scales, up, up_s, m, k, layout, 0, u);
    v3o_nvfp4_page_matvec(act_codes, act_scales, gate, gate_s, m, k, layout, 0, g);
    for (size_t i = 0; i < m; i++) {
        const float sig = 1.0f / (1.0f + v3o_exp_cw(-g[i]));
        out[i] = (g[i] * sig) * u[i];
    }
    free(u);
    free(g);
}
