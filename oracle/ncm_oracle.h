/*
 * CPU oracle for the ncmorph hot path. TEST INFRASTRUCTURE ONLY.
 *
 * This library is the checker: only the test suite, the smoke check and the
 * CPU-baseline leg of the benchmark load it. The product path (the HIP
 * library) never links, loads or calls it.
 *
 * Linear part: a restatement of packages/kernels/root.zig:96-148 and
 * packages/bf16/root.zig:17-37 of the reference (Zig, single-threaded).
 * Pinned bit-exactly by the reference's own known-answer tests
 * (packages/kernels/root.zig:707-770, packages/bf16/root.zig:43-59).
 *
 * RVQ part: the reference has no RVQ code (ROADMAP.md:257-259). This is a
 * restatement of the multiscale residual quantizer described in
 * research/reference/vq_forward_semantics.md:59-82 (nearest code by
 * ||u||^2 + ||c||^2 - 2 u.c, lowest index on ties, codes concatenated level 0
 * first, PROJECT.md:279), in the average-pool / nearest-repeat variant with
 * power-of-two strides. Its fp32 operation order is fixed here and is the
 * contract the GPU path reproduces bit for bit:
 *   pool:  P_1 = x;  P_2s[t] = (P_s[2t] + P_s[2t+1]) * 0.5f
 *   coarse reconstruction at level l, row t':  D = 0; for j < l: D += C_j[code_j]
 *   pooled residual:  u = P_{s_l}[t'] - D
 *   dot / squared norm:  ncmo_dot_fixed (64 strided lanes + halving tree)
 *   dist_k = fmaf(-2, dot(u, c_k), csq_k);  code = lowest k with minimal dist
 *   reconstruction:  recon[t] = sum over l (in order) of C_l[code_l[t / s_l]]
 * The RVQ functions are pinned by f64 brute force, planted codes, tie-break
 * and pooling invariants in the test suite, not by any reference test
 * (none exists).
 */
#ifndef NCM_ORACLE_H
#define NCM_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- bf16 numerics: packages/bf16/root.zig:17-37 ---- */
uint16_t ncmo_bf16_from_f32(float value);
float ncmo_bf16_to_f32(uint16_t bits);
float ncmo_round_bf16(float value); /* packages/kernels/root.zig:10-12 */
void ncmo_bf16_from_f32_array(const float* src, uint16_t* dst, size_t n);
void ncmo_widen_little_endian(float* dst, const uint8_t* src, size_t n);
float ncmo_flush_f32_subnormal(float value); /* root.zig:144-148 */

/* ---- linear: packages/kernels/root.zig ---- */
/* matmul_bf16 / matmul_bf16_bias (:96-142). bias may be NULL.
 * sum_out (nullable) receives the fp32 sum before the final bf16 rounding
 * (after the bias add). Rows [row_begin, row_end) only. */
void ncmo_matmul_bf16_rows(const float* input, const float* weights, const float* bias,
                           float* output, float* sum_out, size_t token_count,
                           size_t input_width, size_t output_width, size_t row_begin,
                           size_t row_end);
void ncmo_matmul_bf16(const float* input, const float* weights, const float* bias,
                      float* output, float* sum_out, size_t token_count, size_t input_width,
                      size_t output_width);
void ncmo_matmul_bf16_mt(const float* input, const float* weights, const float* bias,
                         float* output, float* sum_out, size_t token_count, size_t input_width,
                         size_t output_width, int threads);
/* Same, operands given as bf16 bit patterns (already rounded). */
void ncmo_matmul_bf16_u16_rows(const uint16_t* input, const uint16_t* weights,
                               const uint16_t* bias, float* output, float* sum_out,
                               size_t token_count, size_t input_width, size_t output_width,
                               size_t row_begin, size_t row_end);
/* f32 matmul_reference (:71-93): increasing k, separate multiply and add. */
void ncmo_matmul_reference(const float* input, const float* weights, float* output,
                           size_t token_count, size_t input_width, size_t output_width);
/* f64 dot products and sum |x_k w_k| for the D53 bound (PROJECT.md:506). */
void ncmo_matmul_f64(const float* input, const float* weights, double* output,
                     double* abs_sum, size_t token_count, size_t input_width,
                     size_t output_width);
uint64_t ncmo_fnv1a_bf16_digest(const float* values, size_t n);

/* ---- RVQ ---- */
float ncmo_dot_fixed(const float* u, const uint16_t* c, int64_t d);
float ncmo_sumsq_bf16_fixed(const uint16_t* c, int64_t d);
float ncmo_sumsq_f32_fixed(const float* u, int64_t d);
/* csq[l*v + k] = fixed-order squared norm of codebook row (l, k). */
void ncmo_rvq_csq(const uint16_t* codebooks, int64_t levels, int64_t v, int64_t d,
                  float* csq);
/* Returns 0, or a negative value for an invalid stride schedule. */
int ncmo_rvq_check_strides(int64_t t, int64_t levels, const int32_t* strides);
int64_t ncmo_rvq_codes_per_batch(int64_t t, int64_t levels, const int32_t* strides);
/* Full encode. codes: [b][sum_l t/s_l] int32 (level 0 first).
 * recon (nullable): [b][t][d]. gap (nullable): same layout as codes, the
 * relative gap (e2 - e1) / |e1| of the two smallest full distances
 * e = ||u||^2 + dist (f64). forced (nullable): codes used to build the
 * residual of later levels (teacher forcing); codes still receives the
 * oracle's own argmin. threads: worker threads (0 or 1 = serial). */
int ncmo_rvq_encode(const float* x, int64_t b, int64_t t, int64_t d, int64_t levels,
                    const int32_t* strides, const uint16_t* codebooks, const float* csq,
                    int64_t v, int32_t* codes, float* recon, float* gap,
                    const int32_t* forced, int threads);
/* Level-l codes for selected rows only, given codes of levels < l (from any
 * source). rows: row indices within level l (b * (t/s_l) + t'). */
int ncmo_rvq_level_rows(const float* x, int64_t b, int64_t t, int64_t d, int64_t levels,
                        const int32_t* strides, const uint16_t* codebooks, const float* csq,
                        int64_t v, const int32_t* codes, int64_t level, const int64_t* rows,
                        int64_t n_rows, int32_t* out_codes, float* out_gap, float* out_u);
int ncmo_rvq_decode(const int32_t* codes, int64_t b, int64_t t, int64_t d, int64_t levels,
                    const int32_t* strides, const uint16_t* codebooks, int64_t v,
                    float* recon);
/* Independent f64 restatement used to pin the above: materializes the
 * full-resolution residual r, pools it by plain f64 means, computes f64
 * distances ||u||^2 + ||c||^2 - 2 u.c, lowest index on ties, and updates
 * r -= repeat(q). Returns codes and the f64 relative top-2 gap. */
int ncmo_rvq_encode_f64(const float* x, int64_t b, int64_t t, int64_t d, int64_t levels,
                        const int32_t* strides, const uint16_t* codebooks, int64_t v,
                        int32_t* codes, double* gap, const int32_t* forced);

/* ---- decoder ops around the linear (packages/kernels/root.zig:150-270) ---- */
/* pinned_torch_sum_squares_f32 (root.zig:152-227): 8-lane vectors grouped in
 * rows of four, 4 x 4 x 8 accumulators flushed level by level every
 * 2^level_power row groups, then the row-group tail, the level merge, the
 * vector tail, the row merge and the scalar tail, each a separate fp32
 * product and add in that order. */
float ncmo_sum_squares_pinned(const float* x, size_t n);
/* rms_norm (root.zig:229-242, bf16 = 0) and rms_norm_bf16 (root.zig:246-254,
 * bf16 = 1). n > 0. */
void ncmo_rms_norm(const float* x, const float* weight, float* out, size_t n, float epsilon,
                   int bf16);
/* silu_bf16 (root.zig:265-270): round_bf16(v / (1 + exp(-v))), libm expf. */
void ncmo_silu_bf16(const float* x, float* out, size_t n);
/* The decoder's MLP activation in bf16 mode (src/decoder.zig:210-211):
 * round_bf16(silu_bf16(gate) * up). */
void ncmo_silu_mul_bf16(const float* gate, const float* up, float* out, size_t n);

/* rotate_head (root.zig:615-634): rotate-half RoPE of one head in place;
 * bf16 != 0 rounds the table entries, each product and each sum to bf16. */
void ncmo_rotate_head(float* values, const float* cosine, const float* sine, size_t head_dim,
                      int bf16);
/* causal_mask (root.zig:380-399) for positions 0..count-1; window 0 = none.
 * out[q * key_count + k] = 1 where key k may contribute to query q. */
void ncmo_causal_mask(size_t query_count, size_t key_count, size_t window, uint8_t* out);
/* The attention of attention_impl (root.zig:536-578) after the projections,
 * the optional QK norm and the rotation: per query and head, scores
 * round(round(q.k) * 1/sqrt(head_dim)) (sequential fp32 dot), masked keys
 * -inf, softmax (root.zig:272-284: max, exp(s - max), sequential sum,
 * divide), probabilities rounded to bf16, context round(sum_k p v)
 * (sequential in key order). Key/value head = query head / (q_heads /
 * kv_heads). bf16 = 0: no roundings (the f32 path). Rows of queries and
 * context are [q_heads * head_dim], of keys and values [kv_heads * head_dim]. */
/* RoPE tables, host libm (root.zig:305-348, 636-682; system powf, cosf and
 * sinf as the reference links them). inv has head_dim / 2 entries; the
 * tables are [positions, 2 * half] with each angle's value duplicated into
 * both halves. */
void ncmo_rope_default_frequencies(size_t head_dim, float theta, float* inv);
void ncmo_rope_llama3(size_t head_dim, float theta, float factor, float low_freq_factor,
                      float high_freq_factor, size_t original_max_positions, float* inv);
void ncmo_rope_tables(const float* inv, size_t half, size_t positions, float* cosine,
                      float* sine);
/* block_diagonal_mask (src/ncm_mask.zig:10-42): prefix queries see unpadded
 * prefix keys; a level's queries see unpadded prefix keys and their own
 * level. Returns -1 (InvalidPrefixMask), -2 (InvalidMaskSize) or 0. */
int ncmo_block_diagonal_mask(size_t prefix_length, const size_t* level_lengths, size_t levels,
                             const uint8_t* prefix_pad_mask, size_t pad_len, uint8_t* output,
                             size_t output_len);
void ncmo_attention_core(const float* queries, const float* keys, const float* values,
                         const uint8_t* mask, float* context, size_t tokens, size_t q_heads,
                         size_t kv_heads, size_t head_dim, int bf16);

/* NCM body helpers. */
void ncmo_silu(const float* x, float* out, size_t n);
int ncmo_fill_level_positions(size_t prefix_length, const size_t* level_lengths, size_t levels,
                              int64_t* positions, size_t positions_len);
int ncmo_post_upsample_conv(float* input, const float* weight, const float* bias, size_t rows,
                            size_t width);

#ifdef __cplusplus
}
#endif

#endif
