/*
 * CPU oracle for the ncmorph hot path. TEST INFRASTRUCTURE ONLY: loaded by
 * the test suite, the smoke check and the CPU-baseline leg of the benchmark,
 * never by the product path. Build: oracle/Makefile (-O3 -mfma
 * -ffp-contract=off; every fused multiply-add is an explicit fmaf).
 *
 * Parity status of each function:
 *   bf16 from/to/widen/flush .... pinned (reference KAT vectors + exhaustive)
 *   ncmo_matmul_bf16* ........... pinned (reference KATs root.zig:707-770)
 *   ncmo_matmul_reference ....... pinned (hand-computed KAT root.zig:684-695,
 *                                 D53 bound vs f64)
 *   RVQ (dot, csq, encode, level_rows, decode) ... pinned by mathematics only
 *     (f64 brute force, planted codes, tie-break, pooling invariants), since
 *     the reference has no RVQ implementation or test.
 */
#include "ncm_oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------ */
/* bf16 numerics                                                       */
/* ------------------------------------------------------------------ */

static inline uint32_t f2u(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    return u;
}
static inline float u2f(uint32_t u) {
    float f;
    memcpy(&f, &u, 4);
    return f;
}

/* packages/bf16/root.zig:17-22: RNE, every NaN -> 0x7FC0, no FTZ. */
uint16_t ncmo_bf16_from_f32(float value) {
    uint32_t x = f2u(value);
    if ((x & 0x7FFFFFFFu) > 0x7F800000u) return 0x7FC0u;
    uint32_t bias = 0x7FFFu + ((x >> 16) & 1u);
    return (uint16_t)((x + bias) >> 16);
}

/* packages/bf16/root.zig:25-27: exact widen. */
float ncmo_bf16_to_f32(uint16_t bits) { return u2f((uint32_t)bits << 16); }

/* packages/kernels/root.zig:10-12 */
float ncmo_round_bf16(float value) { return ncmo_bf16_to_f32(ncmo_bf16_from_f32(value)); }

void ncmo_bf16_from_f32_array(const float* src, uint16_t* dst, size_t n) {
    for (size_t i = 0; i < n; ++i) dst[i] = ncmo_bf16_from_f32(src[i]);
}

/* packages/bf16/root.zig:31-37: little-endian bf16 bytes -> f32. */
void ncmo_widen_little_endian(float* dst, const uint8_t* src, size_t n) {
    for (size_t i = 0; i < n; ++i) {
        uint16_t bits = (uint16_t)(src[2 * i] | ((uint16_t)src[2 * i + 1] << 8));
        dst[i] = ncmo_bf16_to_f32(bits);
    }
}

/* packages/kernels/root.zig:144-148: exponent bits zero -> signed zero. */
float ncmo_flush_f32_subnormal(float value) {
    uint32_t bits = f2u(value);
    if ((bits & 0x7F800000u) == 0) return u2f(bits & 0x80000000u);
    return value;
}

/* ------------------------------------------------------------------ */
/* linear                                                              */
/* ------------------------------------------------------------------ */

/* K-block rule of root.zig:112: 512 when K <= 1024, 1024 when K > 1024,
 * never more than K. */
static size_t reduction_block(size_t input_width) {
    size_t b = input_width > 1024 ? 1024 : 512;
    return input_width < b ? input_width : b;
}

#define FTZ ncmo_flush_f32_subnormal

/* root.zig:106-142, for one (token, output) pair. xin/win: f32 values that
 * are rounded to bf16 on use (bf16 values pass through unchanged). */
static float bf16_dot_f32(const float* xin, const float* win, size_t k, size_t kb) {
    float sum = 0.0f;
    for (size_t b0 = 0; b0 < k; b0 += kb) {
        size_t b1 = b0 + kb < k ? b0 + kb : k;
        float partial = 0.0f;
        size_t i = b0;
        for (; i + 1 < b1; i += 2) {
            /* root.zig:124-129: the high element of each pair first. */
            float ih = FTZ(ncmo_round_bf16(xin[i + 1]));
            float wh = FTZ(ncmo_round_bf16(win[i + 1]));
            float il = FTZ(ncmo_round_bf16(xin[i]));
            float wl = FTZ(ncmo_round_bf16(win[i]));
            partial = FTZ(fmaf(ih, wh, partial));
            partial = FTZ(fmaf(il, wl, partial));
        }
        if (i < b1) { /* odd tail, root.zig:131-135 */
            float iv = FTZ(ncmo_round_bf16(xin[i]));
            float wv = FTZ(ncmo_round_bf16(win[i]));
            partial = FTZ(fmaf(iv, wv, partial));
        }
        sum += partial; /* no flush on block sums, root.zig:136 */
    }
    return sum;
}

static float bf16_dot_u16(const uint16_t* xin, const uint16_t* win, size_t k, size_t kb) {
    float sum = 0.0f;
    for (size_t b0 = 0; b0 < k; b0 += kb) {
        size_t b1 = b0 + kb < k ? b0 + kb : k;
        float partial = 0.0f;
        size_t i = b0;
        for (; i + 1 < b1; i += 2) {
            float ih = FTZ(ncmo_bf16_to_f32(xin[i + 1]));
            float wh = FTZ(ncmo_bf16_to_f32(win[i + 1]));
            float il = FTZ(ncmo_bf16_to_f32(xin[i]));
            float wl = FTZ(ncmo_bf16_to_f32(win[i]));
            partial = FTZ(fmaf(ih, wh, partial));
            partial = FTZ(fmaf(il, wl, partial));
        }
        if (i < b1) {
            float iv = FTZ(ncmo_bf16_to_f32(xin[i]));
            float wv = FTZ(ncmo_bf16_to_f32(win[i]));
            partial = FTZ(fmaf(iv, wv, partial));
        }
        sum += partial;
    }
    return sum;
}

void ncmo_matmul_bf16_rows(const float* input, const float* weights, const float* bias,
                           float* output, float* sum_out, size_t token_count,
                           size_t input_width, size_t output_width, size_t row_begin,
                           size_t row_end) {
    (void)token_count;
    size_t kb = reduction_block(input_width);
    for (size_t t = row_begin; t < row_end; ++t) {
        for (size_t o = 0; o < output_width; ++o) {
            float sum = kb ? bf16_dot_f32(input + t * input_width,
                                          weights + o * input_width, input_width, kb)
                           : 0.0f;
            if (bias) sum += ncmo_round_bf16(bias[o]); /* root.zig:138 */
            if (sum_out) sum_out[t * output_width + o] = sum;
            output[t * output_width + o] = ncmo_round_bf16(sum); /* root.zig:139 */
        }
    }
}

void ncmo_matmul_bf16(const float* input, const float* weights, const float* bias,
                      float* output, float* sum_out, size_t token_count, size_t input_width,
                      size_t output_width) {
    ncmo_matmul_bf16_rows(input, weights, bias, output, sum_out, token_count, input_width,
                          output_width, 0, token_count);
}

/* The same arithmetic with the output columns split over `threads` POSIX
 * threads: every element is computed exactly as ncmo_matmul_bf16 computes
 * it, so the results are bit-identical (a speed-up for large checks only). */
struct mm_job {
    const float *input, *weights, *bias;
    float *output, *sum_out;
    size_t token_count, input_width, output_width, o_begin, o_end, kb;
};

static void* mm_worker(void* arg) {
    const struct mm_job* j = (const struct mm_job*)arg;
    for (size_t t = 0; t < j->token_count; ++t) {
        for (size_t o = j->o_begin; o < j->o_end; ++o) {
            float sum = j->kb ? bf16_dot_f32(j->input + t * j->input_width,
                                             j->weights + o * j->input_width, j->input_width,
                                             j->kb)
                              : 0.0f;
            if (j->bias) sum += ncmo_round_bf16(j->bias[o]);
            if (j->sum_out) j->sum_out[t * j->output_width + o] = sum;
            j->output[t * j->output_width + o] = ncmo_round_bf16(sum);
        }
    }
    return NULL;
}

void ncmo_matmul_bf16_mt(const float* input, const float* weights, const float* bias,
                         float* output, float* sum_out, size_t token_count, size_t input_width,
                         size_t output_width, int threads) {
    if (threads < 2 || output_width < 64) {
        ncmo_matmul_bf16(input, weights, bias, output, sum_out, token_count, input_width,
                         output_width);
        return;
    }
    if (threads > 64) threads = 64;
    pthread_t tids[64];
    struct mm_job jobs[64];
    const size_t kb = reduction_block(input_width);
    int started = 0;
    for (int w = 0; w < threads; ++w) {
        const size_t o0 = output_width * (size_t)w / (size_t)threads;
        const size_t o1 = output_width * (size_t)(w + 1) / (size_t)threads;
        jobs[w] = (struct mm_job){input, weights, bias, output, sum_out, token_count,
                                  input_width, output_width, o0, o1, kb};
        if (pthread_create(&tids[w], NULL, mm_worker, &jobs[w]) != 0) {
            mm_worker(&jobs[w]);
            tids[w] = 0;
        } else {
            ++started;
        }
    }
    for (int w = 0; w < threads; ++w)
        if (tids[w]) pthread_join(tids[w], NULL);
    (void)started;
}

void ncmo_matmul_bf16_u16_rows(const uint16_t* input, const uint16_t* weights,
                               const uint16_t* bias, float* output, float* sum_out,
                               size_t token_count, size_t input_width, size_t output_width,
                               size_t row_begin, size_t row_end) {
    (void)token_count;
    size_t kb = reduction_block(input_width);
    for (size_t t = row_begin; t < row_end; ++t) {
        for (size_t o = 0; o < output_width; ++o) {
            float sum = kb ? bf16_dot_u16(input + t * input_width,
                                          weights + o * input_width, input_width, kb)
                           : 0.0f;
            if (bias) sum += ncmo_bf16_to_f32(bias[o]);
            if (sum_out) sum_out[t * output_width + o] = sum;
            output[t * output_width + o] = ncmo_round_bf16(sum);
        }
    }
}

/* root.zig:71-93: increasing k, f32 product then f32 add (no fusion). */
void ncmo_matmul_reference(const float* input, const float* weights, float* output,
                           size_t token_count, size_t input_width, size_t output_width) {
    for (size_t t = 0; t < token_count; ++t)
        for (size_t o = 0; o < output_width; ++o) {
            float sum = 0.0f;
            for (size_t k = 0; k < input_width; ++k) {
                float p = input[t * input_width + k] * weights[o * input_width + k];
                sum += p;
            }
            output[t * output_width + o] = sum;
        }
}

void ncmo_matmul_f64(const float* input, const float* weights, double* output,
                     double* abs_sum, size_t token_count, size_t input_width,
                     size_t output_width) {
    for (size_t t = 0; t < token_count; ++t)
        for (size_t o = 0; o < output_width; ++o) {
            double s = 0.0, a = 0.0;
            for (size_t k = 0; k < input_width; ++k) {
                double p = (double)input[t * input_width + k] *
                           (double)weights[o * input_width + k];
                s += p;
                a += fabs(p);
            }
            output[t * output_width + o] = s;
            if (abs_sum) abs_sum[t * output_width + o] = a;
        }
}

/* FNV-1a-64 over the bf16 bits of each value, root.zig:734-739. */
uint64_t ncmo_fnv1a_bf16_digest(const float* values, size_t n) {
    uint64_t h = 14695981039346656037ull;
    for (size_t i = 0; i < n; ++i) {
        uint16_t bits = (uint16_t)(f2u(values[i]) >> 16);
        h = (h ^ bits) * 1099511628211ull;
    }
    return h;
}

/* ------------------------------------------------------------------ */
/* RVQ                                                                 */
/* ------------------------------------------------------------------ */

/* Fixed fp32 order for a length-d dot product: 64 lanes; lane j owns
 * elements i = 256 m + 4 j + e (m ascending, then e = 0..3) and accumulates
 * them with fmaf from +0; then a halving tree acc[j] += acc[j + off] for
 * off = 32, 16, ..., 1. The GPU computes one such dot per wavefront
 * (lane j loads float4 u[256m + 4j ..]) and reduces with an xor butterfly,
 * which yields the same bits because fp32 addition is commutative. */
float ncmo_dot_fixed(const float* u, const uint16_t* c, int64_t d) {
    float acc[64];
    for (int j = 0; j < 64; ++j) acc[j] = 0.0f;
    for (int64_t m = 0; m * 256 < d; ++m) {
        const float* um = u + m * 256;
        const uint16_t* cm = c + m * 256;
        int64_t rem = d - m * 256;
        if (rem >= 256) {
            for (int e = 0; e < 4; ++e)
                for (int j = 0; j < 64; ++j)
                    acc[j] = fmaf(um[4 * j + e], ncmo_bf16_to_f32(cm[4 * j + e]), acc[j]);
        } else {
            for (int e = 0; e < 4; ++e)
                for (int j = 0; j < 64; ++j)
                    if (4 * j + e < rem)
                        acc[j] = fmaf(um[4 * j + e], ncmo_bf16_to_f32(cm[4 * j + e]), acc[j]);
        }
    }
    for (int off = 32; off >= 1; off >>= 1)
        for (int j = 0; j < off; ++j) acc[j] = acc[j] + acc[j + off];
    return acc[0];
}

float ncmo_sumsq_bf16_fixed(const uint16_t* c, int64_t d) {
    float acc[64];
    for (int j = 0; j < 64; ++j) acc[j] = 0.0f;
    for (int64_t m = 0; m * 256 < d; ++m)
        for (int e = 0; e < 4; ++e)
            for (int j = 0; j < 64; ++j) {
                int64_t i = m * 256 + 4 * j + e;
                if (i < d) {
                    float v = ncmo_bf16_to_f32(c[i]);
                    acc[j] = fmaf(v, v, acc[j]);
                }
            }
    for (int off = 32; off >= 1; off >>= 1)
        for (int j = 0; j < off; ++j) acc[j] = acc[j] + acc[j + off];
    return acc[0];
}

float ncmo_sumsq_f32_fixed(const float* u, int64_t d) {
    float acc[64];
    for (int j = 0; j < 64; ++j) acc[j] = 0.0f;
    for (int64_t m = 0; m * 256 < d; ++m)
        for (int e = 0; e < 4; ++e)
            for (int j = 0; j < 64; ++j) {
                int64_t i = m * 256 + 4 * j + e;
                if (i < d) acc[j] = fmaf(u[i], u[i], acc[j]);
            }
    for (int off = 32; off >= 1; off >>= 1)
        for (int j = 0; j < off; ++j) acc[j] = acc[j] + acc[j + off];
    return acc[0];
}

void ncmo_rvq_csq(const uint16_t* codebooks, int64_t levels, int64_t v, int64_t d,
                  float* csq) {
    for (int64_t r = 0; r < levels * v; ++r) csq[r] = ncmo_sumsq_bf16_fixed(codebooks + r * d, d);
}

static int is_pow2(int64_t s) { return s >= 1 && (s & (s - 1)) == 0; }

int ncmo_rvq_check_strides(int64_t t, int64_t levels, const int32_t* strides) {
    if (levels < 1 || t < 1) return -1;
    for (int64_t l = 0; l < levels; ++l) {
        if (!is_pow2(strides[l])) return -2;
        if (l > 0 && strides[l] > strides[l - 1]) return -3;
    }
    if (t % strides[0] != 0) return -4;
    return 0;
}

int64_t ncmo_rvq_codes_per_batch(int64_t t, int64_t levels, const int32_t* strides) {
    int64_t n = 0;
    for (int64_t l = 0; l < levels; ++l) {
        if (strides[l] < 1) return -1;
        n += t / strides[l];
    }
    return n;
}

static int64_t level_offset(int64_t t, const int32_t* strides, int64_t l) {
    int64_t off = 0;
    for (int64_t j = 0; j < l; ++j) off += t / strides[j];
    return off;
}

/* P_s for one row: the pairwise tree over x rows [t0, t0 + s). */
static void pooled_row(const float* x, int64_t d, int64_t t0, int64_t s, float* out,
                       float* scratch) {
    if (s == 1) {
        memcpy(out, x + t0 * d, (size_t)d * sizeof(float));
        return;
    }
    /* scratch holds s rows; halve in place, pairing (2t, 2t+1). */
    memcpy(scratch, x + t0 * d, (size_t)(s * d) * sizeof(float));
    for (int64_t n = s; n > 1; n >>= 1)
        for (int64_t r = 0; r < n / 2; ++r)
            for (int64_t i = 0; i < d; ++i)
                scratch[r * d + i] = (scratch[2 * r * d + i] + scratch[(2 * r + 1) * d + i]) * 0.5f;
    memcpy(out, scratch, (size_t)d * sizeof(float));
}

/* u = P_{s_l}[row] - (sum over j < l, in order, of C_j[code_j]) */
static void residual_row(const float* x, int64_t t, int64_t d, const int32_t* strides,
                         const uint16_t* codebooks, int64_t v, const int32_t* codes_b,
                         int64_t l, int64_t tp, float* u, float* dacc, float* scratch) {
    int64_t s = strides[l];
    pooled_row(x, d, tp * s, s, u, scratch);
    for (int64_t i = 0; i < d; ++i) dacc[i] = 0.0f;
    int64_t off = 0;
    for (int64_t j = 0; j < l; ++j) {
        int64_t rj = (tp * s) / strides[j];
        int32_t k = codes_b[off + rj];
        const uint16_t* c = codebooks + ((int64_t)j * v + k) * d;
        for (int64_t i = 0; i < d; ++i) dacc[i] = dacc[i] + ncmo_bf16_to_f32(c[i]);
        off += t / strides[j];
    }
    for (int64_t i = 0; i < d; ++i) u[i] = u[i] - dacc[i];
}

/* argmin over all codes of fmaf(-2, dot, csq); lowest index on ties;
 * relative gap of the two smallest full distances in f64. */
static void nearest_code(const float* u, int64_t d, const uint16_t* cb_level,
                         const float* csq_level, int64_t v, int32_t* code, float* gap) {
    float best = INFINITY, second = INFINITY;
    int32_t best_k = 0;
    for (int64_t k = 0; k < v; ++k) {
        float dot = ncmo_dot_fixed(u, cb_level + k * d, d);
        float dist = fmaf(-2.0f, dot, csq_level[k]);
        if (dist < best) {
            second = best;
            best = dist;
            best_k = (int32_t)k;
        } else if (dist < second) {
            second = dist;
        }
    }
    *code = best_k;
    if (gap) {
        double un = 0.0;
        for (int64_t i = 0; i < d; ++i) un += (double)u[i] * (double)u[i];
        double e1 = un + (double)best, e2 = un + (double)second;
        double g = (v < 2 || isinf(second)) ? INFINITY : (e2 - e1) / fmax(fabs(e1), 1e-300);
        *gap = (float)g;
    }
}

typedef struct {
    const float* x;
    int64_t b, t, d, v, l;
    const int32_t* strides;
    const uint16_t* codebooks;
    const float* csq;
    const int32_t* resid_codes; /* codes used for the residual of level l */
    int32_t* codes;             /* output codes (own argmin) */
    float* gap;
    int64_t row_begin, row_end, total;
} level_job_t;

static void* level_worker(void* arg) {
    level_job_t* j = (level_job_t*)arg;
    int64_t s = j->strides[j->l];
    int64_t per_b = j->t / s;
    int64_t off = level_offset(j->t, j->strides, j->l);
    float* u = (float*)malloc((size_t)j->d * sizeof(float));
    float* dacc = (float*)malloc((size_t)j->d * sizeof(float));
    float* scratch = (float*)malloc((size_t)(s * j->d) * sizeof(float));
    const uint16_t* cbl = j->codebooks + j->l * j->v * j->d;
    const float* csql = j->csq + j->l * j->v;
    for (int64_t r = j->row_begin; r < j->row_end; ++r) {
        int64_t bb = r / per_b, tp = r % per_b;
        residual_row(j->x + bb * j->t * j->d, j->t, j->d, j->strides, j->codebooks, j->v,
                     j->resid_codes + bb * j->total, j->l, tp, u, dacc, scratch);
        nearest_code(u, j->d, cbl, csql, j->v, &j->codes[bb * j->total + off + tp],
                     j->gap ? &j->gap[bb * j->total + off + tp] : NULL);
    }
    free(u);
    free(dacc);
    free(scratch);
    return NULL;
}

int ncmo_rvq_encode(const float* x, int64_t b, int64_t t, int64_t d, int64_t levels,
                    const int32_t* strides, const uint16_t* codebooks, const float* csq,
                    int64_t v, int32_t* codes, float* recon, float* gap,
                    const int32_t* forced, int threads) {
    int rc = ncmo_rvq_check_strides(t, levels, strides);
    if (rc) return rc;
    if (b < 1 || d < 1 || v < 1) return -5;
    int64_t total = ncmo_rvq_codes_per_batch(t, levels, strides);
    if (threads < 1) threads = 1;
    /* Residual codes: the oracle's own codes, or the forced ones. */
    const int32_t* resid = forced ? forced : codes;
    for (int64_t l = 0; l < levels; ++l) {
        int64_t rows = b * (t / strides[l]);
        int nt = threads;
        if (nt > rows) nt = (int)rows;
        level_job_t* jobs = (level_job_t*)calloc((size_t)nt, sizeof(level_job_t));
        pthread_t* tids = (pthread_t*)calloc((size_t)nt, sizeof(pthread_t));
        for (int w = 0; w < nt; ++w) {
            level_job_t* j = &jobs[w];
            j->x = x; j->b = b; j->t = t; j->d = d; j->v = v; j->l = l;
            j->strides = strides; j->codebooks = codebooks; j->csq = csq;
            j->resid_codes = resid; j->codes = codes; j->gap = gap; j->total = total;
            j->row_begin = rows * w / nt;
            j->row_end = rows * (w + 1) / nt;
        }
        if (nt == 1) {
            level_worker(&jobs[0]);
        } else {
            for (int w = 0; w < nt; ++w) pthread_create(&tids[w], NULL, level_worker, &jobs[w]);
            for (int w = 0; w < nt; ++w) pthread_join(tids[w], NULL);
        }
        free(jobs);
        free(tids);
    }
    if (recon) return ncmo_rvq_decode(forced ? forced : codes, b, t, d, levels, strides,
                                      codebooks, v, recon);
    return 0;
}

int ncmo_rvq_level_rows(const float* x, int64_t b, int64_t t, int64_t d, int64_t levels,
                        const int32_t* strides, const uint16_t* codebooks, const float* csq,
                        int64_t v, const int32_t* codes, int64_t level, const int64_t* rows,
                        int64_t n_rows, int32_t* out_codes, float* out_gap, float* out_u) {
    int rc = ncmo_rvq_check_strides(t, levels, strides);
    if (rc) return rc;
    if (level < 0 || level >= levels) return -6;
    int64_t s = strides[level];
    int64_t per_b = t / s;
    int64_t total = ncmo_rvq_codes_per_batch(t, levels, strides);
    float* u = (float*)malloc((size_t)d * sizeof(float));
    float* dacc = (float*)malloc((size_t)d * sizeof(float));
    float* scratch = (float*)malloc((size_t)(s * d) * sizeof(float));
    for (int64_t i = 0; i < n_rows; ++i) {
        int64_t r = rows[i];
        if (r < 0 || r >= b * per_b) { rc = -7; break; }
        int64_t bb = r / per_b, tp = r % per_b;
        residual_row(x + bb * t * d, t, d, strides, codebooks, v, codes + bb * total, level, tp,
                     u, dacc, scratch);
        if (out_u) memcpy(out_u + i * d, u, (size_t)d * sizeof(float));
        nearest_code(u, d, codebooks + level * v * d, csq + level * v, v, &out_codes[i],
                     out_gap ? &out_gap[i] : NULL);
    }
    free(u);
    free(dacc);
    free(scratch);
    return rc;
}

int ncmo_rvq_decode(const int32_t* codes, int64_t b, int64_t t, int64_t d, int64_t levels,
                    const int32_t* strides, const uint16_t* codebooks, int64_t v,
                    float* recon) {
    int rc = ncmo_rvq_check_strides(t, levels, strides);
    if (rc) return rc;
    int64_t total = ncmo_rvq_codes_per_batch(t, levels, strides);
    for (int64_t bb = 0; bb < b; ++bb)
        for (int64_t tt = 0; tt < t; ++tt) {
            float* out = recon + (bb * t + tt) * d;
            for (int64_t i = 0; i < d; ++i) out[i] = 0.0f;
            int64_t off = 0;
            for (int64_t l = 0; l < levels; ++l) {
                int32_t k = codes[bb * total + off + tt / strides[l]];
                if (k < 0 || k >= v) return -8;
                const uint16_t* c = codebooks + (l * v + k) * d;
                for (int64_t i = 0; i < d; ++i) out[i] = out[i] + ncmo_bf16_to_f32(c[i]);
                off += t / strides[l];
            }
        }
    return 0;
}

int ncmo_rvq_encode_f64(const float* x, int64_t b, int64_t t, int64_t d, int64_t levels,
                        const int32_t* strides, const uint16_t* codebooks, int64_t v,
                        int32_t* codes, double* gap, const int32_t* forced) {
    /* Strides need only divide t here: the residual is materialized. */
    if (levels < 1) return -1;
    for (int64_t l = 0; l < levels; ++l)
        if (strides[l] < 1 || t % strides[l] != 0) return -4;
    int64_t total = 0;
    for (int64_t l = 0; l < levels; ++l) total += t / strides[l];
    double* r = (double*)malloc((size_t)(b * t * d) * sizeof(double));
    double* u = (double*)malloc((size_t)d * sizeof(double));
    double* cn = (double*)malloc((size_t)v * sizeof(double));
    for (int64_t i = 0; i < b * t * d; ++i) r[i] = (double)x[i];
    int64_t off = 0;
    for (int64_t l = 0; l < levels; ++l) {
        int64_t s = strides[l], per_b = t / s;
        const uint16_t* cbl = codebooks + l * v * d;
        for (int64_t k = 0; k < v; ++k) {
            double a = 0.0;
            for (int64_t i = 0; i < d; ++i) {
                double c = (double)ncmo_bf16_to_f32(cbl[k * d + i]);
                a += c * c;
            }
            cn[k] = a;
        }
        for (int64_t bb = 0; bb < b; ++bb)
            for (int64_t tp = 0; tp < per_b; ++tp) {
                for (int64_t i = 0; i < d; ++i) {
                    double a = 0.0;
                    for (int64_t q = 0; q < s; ++q) a += r[(bb * t + tp * s + q) * d + i];
                    u[i] = a / (double)s;
                }
                double un = 0.0;
                for (int64_t i = 0; i < d; ++i) un += u[i] * u[i];
                double best = INFINITY, second = INFINITY;
                int32_t bk = 0;
                for (int64_t k = 0; k < v; ++k) {
                    double dot = 0.0;
                    for (int64_t i = 0; i < d; ++i)
                        dot += u[i] * (double)ncmo_bf16_to_f32(cbl[k * d + i]);
                    double e = un + cn[k] - 2.0 * dot;
                    if (e < best) {
                        second = best;
                        best = e;
                        bk = (int32_t)k;
                    } else if (e < second) {
                        second = e;
                    }
                }
                int64_t ci = bb * total + off + tp;
                codes[ci] = bk;
                if (gap) gap[ci] = (v < 2) ? INFINITY : (second - best) / fmax(fabs(best), 1e-300);
            }
        for (int64_t bb = 0; bb < b; ++bb)
            for (int64_t tt = 0; tt < t; ++tt) {
                int64_t ci = bb * total + off + tt / s;
                int32_t k = forced ? forced[ci] : codes[ci];
                for (int64_t i = 0; i < d; ++i)
                    r[(bb * t + tt) * d + i] -= (double)ncmo_bf16_to_f32(cbl[k * d + i]);
            }
        off += per_b;
    }
    free(r);
    free(u);
    free(cn);
    return 0;
}

/* ------------------------------------------------------------------ */
/* Decoder ops around the linear                                      */
/* ------------------------------------------------------------------ */

float ncmo_sum_squares_pinned(const float* x, size_t n) {
    enum { W = 8 };
    const size_t vectors = n / W;
    const size_t groups = vectors / 4; /* row groups of four vectors */
    size_t lg = 0, lim = 1;
    while (lim < groups) {
        ++lg;
        lim *= 2;
    }
    const size_t power = lg / 4 > 4 ? lg / 4 : 4;
    const size_t step = (size_t)1 << power;
    const size_t mask = step - 1;
    float acc[4][4][W];
    memset(acc, 0, sizeof(acc));
    size_t g = 0;
    while (g + step <= groups) {
        for (size_t s = 0; s < step; ++s)
            for (int r = 0; r < 4; ++r)
                for (int l = 0; l < W; ++l) {
                    const float v = x[((g + s) * 4 + r) * W + l];
                    const float sq = v * v;
                    acc[0][r][l] = acc[0][r][l] + sq;
                }
        g += step;
        for (int lev = 1; lev < 4; ++lev) {
            for (int r = 0; r < 4; ++r)
                for (int l = 0; l < W; ++l) {
                    acc[lev][r][l] = acc[lev][r][l] + acc[lev - 1][r][l];
                    acc[lev - 1][r][l] = 0.0f;
                }
            if ((g & (mask << (lev * power))) != 0) break;
        }
    }
    for (; g < groups; ++g)
        for (int r = 0; r < 4; ++r)
            for (int l = 0; l < W; ++l) {
                const float v = x[(g * 4 + r) * W + l];
                const float sq = v * v;
                acc[0][r][l] = acc[0][r][l] + sq;
            }
    for (int lev = 1; lev < 4; ++lev)
        for (int r = 0; r < 4; ++r)
            for (int l = 0; l < W; ++l) acc[0][r][l] = acc[0][r][l] + acc[lev][r][l];
    for (size_t vi = groups * 4; vi < vectors; ++vi)
        for (int l = 0; l < W; ++l) {
            const float v = x[vi * W + l];
            const float sq = v * v;
            acc[0][0][l] = acc[0][0][l] + sq;
        }
    float vs[W];
    for (int l = 0; l < W; ++l) vs[l] = acc[0][0][l];
    for (int r = 1; r < 4; ++r)
        for (int l = 0; l < W; ++l) vs[l] = vs[l] + acc[0][r][l];
    float sum = 0.0f;
    for (size_t i = vectors * W; i < n; ++i) {
        const float sq = x[i] * x[i];
        sum = sum + sq;
    }
    for (int l = 0; l < W; ++l) sum = sum + vs[l];
    return sum;
}

void ncmo_rms_norm(const float* x, const float* weight, float* out, size_t n, float epsilon,
                   int bf16) {
    const float ss = ncmo_sum_squares_pinned(x, n);
    const float mean = ss / (float)n;
    const float inv = 1.0f / sqrtf(mean + epsilon);
    for (size_t i = 0; i < n; ++i) {
        if (bf16) {
            const float normalized = ncmo_round_bf16(x[i] * inv);
            out[i] = ncmo_round_bf16(normalized * ncmo_round_bf16(weight[i]));
        } else {
            const float normalized = x[i] * inv;
            out[i] = normalized * weight[i];
        }
    }
}

void ncmo_silu_bf16(const float* x, float* out, size_t n) {
    for (size_t i = 0; i < n; ++i) {
        const float v = x[i];
        out[i] = ncmo_round_bf16(v / (1.0f + expf(-v)));
    }
}

/* kernels.silu (packages/kernels/root.zig:255-261): value * (1 / (1 +
 * exp(-value))), f32 mode. libm expf stands in for Zig's std.math.exp (not
 * bit-pinned; see the decoder ops). */
void ncmo_silu(const float* x, float* out, size_t n) {
    for (size_t i = 0; i < n; ++i) {
        const float v = x[i];
        const float sigmoid = 1.0f / (1.0f + expf(-v));
        out[i] = v * sigmoid;
    }
}

void ncmo_silu_mul_bf16(const float* gate, const float* up, float* out, size_t n) {
    for (size_t i = 0; i < n; ++i) {
        const float v = gate[i];
        const float a = ncmo_round_bf16(v / (1.0f + expf(-v)));
        out[i] = ncmo_round_bf16(a * up[i]);
    }
}

static float maybe_round(float v, int bf16) { return bf16 ? ncmo_round_bf16(v) : v; }

void ncmo_rotate_head(float* values, const float* cosine, const float* sine, size_t head_dim,
                      int bf16) {
    const size_t half = head_dim / 2;
    for (size_t i = 0; i < half; ++i) {
        const float first = values[i];
        const float second = values[i + half];
        const float cos_first = maybe_round(cosine[i], bf16);
        const float sin_first = maybe_round(sine[i], bf16);
        const float cos_second = maybe_round(cosine[i + half], bf16);
        const float sin_second = maybe_round(sine[i + half], bf16);
        const float left = maybe_round(first * cos_first, bf16);
        const float right = maybe_round(-second * sin_first, bf16);
        const float right2 = maybe_round(first * sin_second, bf16);
        const float left2 = maybe_round(second * cos_second, bf16);
        values[i] = maybe_round(left + right, bf16);
        values[i + half] = maybe_round(left2 + right2, bf16);
    }
}

void ncmo_causal_mask(size_t query_count, size_t key_count, size_t window, uint8_t* out) {
    for (size_t q = 0; q < query_count; ++q)
        for (size_t k = 0; k < key_count; ++k) {
            const int causal = k <= q;
            const int in_window = window == 0 || q < window || k > q - window;
            out[q * key_count + k] = (uint8_t)(causal && in_window);
        }
}

void ncmo_attention_core(const float* queries, const float* keys, const float* values,
                         const uint8_t* mask, float* context, size_t tokens, size_t q_heads,
                         size_t kv_heads, size_t head_dim, int bf16) {
    const size_t qw = q_heads * head_dim, kvw = kv_heads * head_dim;
    const size_t group = q_heads / kv_heads;
    const float scale = 1.0f / sqrtf((float)head_dim);
    float* scores = (float*)malloc(tokens * sizeof(float));
    float* probs = (float*)malloc(tokens * sizeof(float));
    for (size_t qi = 0; qi < tokens; ++qi)
        for (size_t h = 0; h < q_heads; ++h) {
            const float* q = queries + qi * qw + h * head_dim;
            const size_t kvh = h / group;
            int any = 0;
            for (size_t ki = 0; ki < tokens; ++ki) {
                if (!mask[qi * tokens + ki]) {
                    scores[ki] = -INFINITY;
                    continue;
                }
                any = 1;
                const float* k = keys + ki * kvw + kvh * head_dim;
                float score = 0.0f;
                for (size_t d = 0; d < head_dim; ++d) {
                    const float p = q[d] * k[d];
                    score = score + p;
                }
                const float sv = maybe_round(score, bf16);
                scores[ki] = maybe_round(sv * scale, bf16);
            }
            if (any) {
                float mx = scores[0];
                for (size_t ki = 1; ki < tokens; ++ki) mx = scores[ki] > mx ? scores[ki] : mx;
                float sum = 0.0f;
                for (size_t ki = 0; ki < tokens; ++ki) {
                    probs[ki] = expf(scores[ki] - mx);
                    sum = sum + probs[ki];
                }
                for (size_t ki = 0; ki < tokens; ++ki) probs[ki] = probs[ki] / sum;
                if (bf16)
                    for (size_t ki = 0; ki < tokens; ++ki) probs[ki] = ncmo_round_bf16(probs[ki]);
            } else {
                for (size_t ki = 0; ki < tokens; ++ki) probs[ki] = 0.0f;
            }
            float* out = context + qi * qw + h * head_dim;
            for (size_t d = 0; d < head_dim; ++d) {
                float sum = 0.0f;
                for (size_t ki = 0; ki < tokens; ++ki) {
                    const float p = probs[ki] * values[ki * kvw + kvh * head_dim + d];
                    sum = sum + p;
                }
                out[d] = maybe_round(sum, bf16);
            }
        }
    free(scores);
    free(probs);
}

void ncmo_rope_default_frequencies(size_t head_dim, float theta, float* inv) {
    const float hd = (float)head_dim;
    for (size_t i = 0; i < head_dim / 2; ++i) {
        const float exponent = (float)(2 * i) / hd;
        inv[i] = 1.0f / powf(theta, exponent);
    }
}

void ncmo_rope_llama3(size_t head_dim, float theta, float factor, float low_freq_factor,
                      float high_freq_factor, size_t original_max_positions, float* inv) {
    ncmo_rope_default_frequencies(head_dim, theta, inv);
    const float old_context_len = (float)original_max_positions;
    const float low_wavelen = (float)((double)original_max_positions / (double)low_freq_factor);
    const float high_wavelen = (float)((double)original_max_positions / (double)high_freq_factor);
    const float two_pi = (float)(2.0 * 3.14159265358979323846);
    for (size_t i = 0; i < head_dim / 2; ++i) {
        const float f = inv[i];
        const float wavelen = two_pi / f;
        const float llama = wavelen > low_wavelen ? f / factor : f;
        const float smooth =
            (old_context_len / wavelen - low_freq_factor) / (high_freq_factor - low_freq_factor);
        const float a = (1.0f - smooth) * llama;
        const float b = smooth * llama;
        const float smoothed = a / factor + b;
        const int medium = !(wavelen < high_wavelen) && !(wavelen > low_wavelen);
        inv[i] = medium ? smoothed : llama;
    }
}

void ncmo_rope_tables(const float* inv, size_t half, size_t positions, float* cosine,
                      float* sine) {
    const size_t hd = 2 * half;
    for (size_t p = 0; p < positions; ++p) {
        const float pf = (float)p;
        for (size_t i = 0; i < half; ++i) {
            const float angle = pf * inv[i];
            const float c = cosf(angle), s = sinf(angle);
            cosine[p * hd + i] = c;
            cosine[p * hd + half + i] = c;
            sine[p * hd + i] = s;
            sine[p * hd + half + i] = s;
        }
    }
}

int ncmo_block_diagonal_mask(size_t prefix_length, const size_t* level_lengths, size_t levels,
                             const uint8_t* prefix_pad_mask, size_t pad_len, uint8_t* output,
                             size_t output_len) {
    if (pad_len != 0 && pad_len != prefix_length) return -1; /* InvalidPrefixMask */
    size_t target = 0;
    for (size_t l = 0; l < levels; ++l) target += level_lengths[l];
    const size_t seq = prefix_length + target;
    if (output_len != seq * seq) return -2; /* InvalidMaskSize */
    memset(output, 0, output_len);
    for (size_t q = 0; q < prefix_length; ++q)
        for (size_t k = 0; k < prefix_length; ++k)
            output[q * seq + k] = !(pad_len && prefix_pad_mask[k]);
    size_t off = prefix_length;
    for (size_t l = 0; l < levels; ++l) {
        for (size_t q = off; q < off + level_lengths[l]; ++q) {
            for (size_t k = 0; k < prefix_length; ++k)
                output[q * seq + k] = !(pad_len && prefix_pad_mask[k]);
            for (size_t k = off; k < off + level_lengths[l]; ++k) output[q * seq + k] = 1;
        }
        off += level_lengths[l];
    }
    return 0;
}

/* ------------------------------------------------------------------ */
/* NCM body helpers (src/ncm_position.zig, src/ncm_model.zig)          */
/* ------------------------------------------------------------------ */

/* fill_level_positions (src/ncm_position.zig:11-22): the prefix takes
 * 0 .. P-1 and every level restarts at 0. -1 = InvalidPositionBuffer. */
int ncmo_fill_level_positions(size_t prefix_length, const size_t* level_lengths, size_t levels,
                              int64_t* positions, size_t positions_len) {
    size_t total = prefix_length;
    for (size_t l = 0; l < levels; ++l) total += level_lengths[l];
    if (positions_len != total) return -1;
    for (size_t p = 0; p < prefix_length; ++p) positions[p] = (int64_t)p;
    size_t off = prefix_length;
    for (size_t l = 0; l < levels; ++l) {
        for (size_t p = 0; p < level_lengths[l]; ++p) positions[off + p] = (int64_t)p;
        off += level_lengths[l];
    }
    return 0;
}

/* apply_post_upsample_conv (src/ncm_model.zig:296-326) on one level chunk
 * [rows, width], in place: value = bias[o], then for every input channel and
 * kernel tap in that order value += weight[o][i][k] * input[p + k - 1][i]
 * (taps outside the chunk skipped; separate multiply and add), and
 * output = input + value. weight: [width][width][3]. -1 on a bad size. */
int ncmo_post_upsample_conv(float* input, const float* weight, const float* bias, size_t rows,
                            size_t width) {
    if (rows == 0 || width == 0) return 0;
    float* out = (float*)malloc(rows * width * sizeof(float));
    if (!out) return -2;
    for (size_t p = 0; p < rows; ++p) {
        for (size_t o = 0; o < width; ++o) {
            float value = bias[o];
            for (size_t i = 0; i < width; ++i) {
                for (size_t k = 0; k < 3; ++k) {
                    const long ip = (long)p + (long)k - 1;
                    if (ip < 0 || ip >= (long)rows) continue;
                    const float prod = weight[o * width * 3 + i * 3 + k] * input[(size_t)ip * width + i];
                    value = value + prod;
                }
            }
            out[p * width + o] = input[p * width + o] + value;
        }
    }
    memcpy(input, out, rows * width * sizeof(float));
    free(out);
    return 0;
}
