/*
 * ncmorph_amd: MI355X (gfx950) implementation of ncmorph's data-parallel hot
 * path behind a plain C ABI. No HIP or torch types cross this boundary:
 * pointers, sizes, int status codes and an opaque context.
 *
 * Two groups of entry points:
 *   1. Drop-in replacements for the reference's Zig `kernels` functions
 *      (host slices in, host slices out, synchronous). A Zig wrapper that
 *      @cImport()s this header keeps the reference signatures and panics on
 *      a nonzero status, as the reference panics on its asserts.
 *   2. Device-resident, stream-ordered entry points (the benchmarked path):
 *      device pointers, bf16 operands as uint16_t bit patterns, fp32 outputs.
 *
 * Status: 0 on success, a negative NCM_E_* value on failure; no entry point
 * aborts. Device entry points are asynchronous on the context's stream.
 *
 * Layouts are row-major. A linear's weights are [out, in] (the reference's
 * layout, packages/kernels/root.zig:57-58). RVQ codebooks are
 * [levels][v][d] bf16; codes are int32 [b][sum_l t/s_l], level 0 first.
 */
#ifndef NCMORPH_AMD_H
#define NCMORPH_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
    NCM_OK = 0,
    NCM_E_NULL = -1,      /* a required pointer is NULL */
    NCM_E_SHAPE = -2,     /* dimensions inconsistent or unsupported */
    NCM_E_LENGTH = -3,    /* a slice length does not match the dimensions */
    NCM_E_HIP = -4,       /* a HIP runtime call failed */
    NCM_E_NOMEM = -5,     /* device or host allocation failed */
    NCM_E_DEVICE = -6,    /* no usable gfx950 device */
    NCM_E_ARG = -7,       /* an argument value is out of range */
    NCM_E_FORMAT = -8,    /* malformed file or header; ncm_last_error() names
                             the reference's error (e.g. "InvalidOffsets") */
    NCM_E_SCRATCH = -9    /* the call needs more than the fixed scratch of an
                             allocation-free entry point holds */
};

/* Linear output modes. */
enum {
    NCM_OUT_F32 = 0,      /* fp32 accumulator, written as float */
    NCM_OUT_BF16_F32 = 1, /* round_bf16(flush(sum)) written as float (the
                             reference's output contract, root.zig:139) */
    NCM_OUT_BF16 = 2      /* round_bf16(flush(sum)) written as uint16 bits */
};

typedef struct ncm_ctx ncm_ctx_t;

/* Human-readable text for a status code. Never NULL. */
const char* ncm_status_string(int status);
/* Text of the last HIP error seen by this thread ("" if none). */
const char* ncm_last_error(void);

/* Context: one device, one stream, cached workspace. Not thread-safe: use
 * one context per host thread. */
int ncm_init(int device, ncm_ctx_t** out);
int ncm_destroy(ncm_ctx_t* ctx);
/* Route the context's work to a stream (a hipStream_t passed as void*;
 * NULL is HIP's default stream). A new context uses a non-blocking stream
 * of its own. The context's entry points share one device workspace: when
 * the stream changes, work queued on the new stream waits for the work
 * already queued on the previous one. */
int ncm_set_stream(ncm_ctx_t* ctx, void* stream);
void* ncm_get_stream(ncm_ctx_t* ctx);
int ncm_synchronize(ncm_ctx_t* ctx);

/* ===================================================================== */
/* 1. Drop-in replacements (host memory, synchronous)                     */
/* ===================================================================== */

/* Replaces `kernels.matmul_bf16` (packages/kernels/root.zig:96-98):
 * output[t, o] = round_bf16(sum_k bf16(input[t, k]) * bf16(weights[o, k])),
 * fp32 accumulation. Operands are rounded to bf16 (RNE, subnormals flushed,
 * as root.zig:124-135 do) on the device. Lengths are the Zig slice lengths
 * and must equal the products of the dimensions (root.zig:107-109).
 * Uses the calling thread's default context on device 0. */
int ncm_matmul_bf16(const float* input, size_t input_len, const float* weights,
                    size_t weights_len, float* output, size_t output_len,
                    size_t token_count, size_t input_width, size_t output_width);

/* Replaces `kernels.matmul_bf16_bias` (packages/kernels/root.zig:102-104):
 * the bias (rounded to bf16) is added to the fp32 sum before the output
 * rounding (root.zig:138). bias_len must equal output_width (:110). */
int ncm_matmul_bf16_bias(const float* input, size_t input_len, const float* weights,
                         size_t weights_len, const float* bias, size_t bias_len,
                         float* output, size_t output_len, size_t token_count,
                         size_t input_width, size_t output_width);

/* `kernels.matmul_bf16` and `matmul_bf16_bias` (packages/kernels/root.zig:
 * 96-142) with the reference's own arithmetic, bit for bit: per output, fp32
 * fma chains over bf16 operand pairs (x[i+1] w[i+1] first, then x[i] w[i]),
 * operands and every partial flushed (root.zig:144-148), blocks of 512
 * (1024 above K = 1024) summed in order, the bias added, one bf16 rounding.
 * Same arguments and errors as the two drop-ins above; VALU arithmetic, for
 * callers whose acceptance gates compare bf16 logits with the reference's
 * (its B9 and C2-C5 checks, src/loader.zig:778-783, :1385-1400), not for
 * speed. */
int ncm_matmul_bf16_exact(const float* input, size_t input_len, const float* weights,
                          size_t weights_len, float* output, size_t output_len,
                          size_t token_count, size_t input_width, size_t output_width);
int ncm_matmul_bf16_bias_exact(const float* input, size_t input_len, const float* weights,
                               size_t weights_len, const float* bias, size_t bias_len,
                               float* output, size_t output_len, size_t token_count,
                               size_t input_width, size_t output_width);

/* Replaces `kernels.matmul` (packages/kernels/root.zig:25-65): fp32
 * output[t, o] = sum_k input[t, k] * weights[o, k] on the fp32 MFMA. The
 * reference accumulates in increasing k (root.zig:55-58); the MFMA order
 * differs, and both meet the reference's own contract
 * |y - y_f64| <= (input_width + 1) 2^-24 sum |x w| (root.zig:836-865).
 * Host pointers; lengths as in root.zig:32-34. */
int ncm_matmul_f32(const float* input, size_t input_len, const float* weights,
                   size_t weights_len, float* output, size_t output_len, size_t token_count,
                   size_t input_width, size_t output_width);

/* Replaces `kernels.round_bf16` (packages/kernels/root.zig:10-12) and
 * `bf16_t.from_f32` (packages/bf16/root.zig:17-22) for whole buffers:
 * RNE, every NaN -> 0x7FC0, no flush. Host pointers. */
int ncm_round_bf16(const float* values, float* out, size_t n);

/* Replaces `kernels.rms_norm_bf16` (packages/kernels/root.zig:246-254): the
 * sum of squares in the reference's pinned order (root.zig:152-227), then
 * round_bf16(round_bf16(x * inverse_rms) * round_bf16(weight)); bit-identical
 * to the reference. One nonempty vector; lengths as root.zig:247. */
int ncm_rms_norm_bf16(const float* input, size_t input_len, const float* weight,
                      size_t weight_len, float* output, size_t output_len, float epsilon);

/* Replaces `kernels.silu_bf16` (packages/kernels/root.zig:265-270):
 * round_bf16(v / (1 + exp(-v))). exp is the device's expf, so a result can
 * differ from the reference's by one bf16 step where the f32 quotient lies
 * next to a rounding boundary. */
int ncm_silu_bf16(const float* input, size_t input_len, float* output, size_t output_len);

/* ===================================================================== */
/* 2. Device-resident entry points (stream-ordered)                        */
/* ===================================================================== */

/* y[m, n] = sum_k x[m, k] * w[n, k] (+ bias[n]), fp32 accumulation on bf16
 * MFMA. x: bf16 [m, k]; w: bf16 [n, k]; bias: bf16 [n] or NULL;
 * y: float [m, n] (out_mode F32 or BF16_F32) or uint16 [m, n] (BF16).
 * Requires k % 8 == 0 and 16-byte aligned x and w.
 * Device counterpart of matmul_bf16_impl (packages/kernels/root.zig:106-142)
 * with the accumulation order of the MFMA instead of oneDNN's pair order;
 * results agree with the reference's fp32 sum within rel 1e-2 / abs 1e-3. */
int ncm_linear_bf16(ncm_ctx_t* ctx, const uint16_t* x, const uint16_t* w,
                    const uint16_t* bias, void* y, int64_t m, int64_t k, int64_t n,
                    int out_mode);

/* ncm_linear_bf16 in the reference's arithmetic bit for bit (the pair-order
 * fma chains of ncm_matmul_bf16_exact; bf16 operand subnormals are flushed
 * in the kernel): out_mode BF16_F32 gives matmul_bf16_impl's output
 * (packages/kernels/root.zig:106-142), F32 its fp32 sum before the output
 * rounding (bias included). Any k >= 0 with row stride k; no alignment
 * requirement. VALU arithmetic, not the benchmarked path. */
int ncm_linear_bf16_exact(ncm_ctx_t* ctx, const uint16_t* x, const uint16_t* w,
                          const uint16_t* bias, void* y, int64_t m, int64_t k, int64_t n,
                          int out_mode);

/* y = residual + ncm_linear_bf16(x, w, bias): the projection and the
 * residual add that follows it in the decoder layer (add_rows,
 * src/decoder.zig:279-282, after the o and down projections at
 * src/decoder.zig:199-200 and 213-214) in one pass. residual: float [m, n].
 * out_mode F32: residual + value in fp32 (the reference's fp32 mode).
 * BF16_F32 / BF16: round_bf16(residual + round_bf16(value)), the bf16 mode's
 * add of the bf16-rounded projection. residual may equal y for F32 and
 * BF16_F32 (in-place update of the hidden state), not for BF16. Same shape and
 * alignment rules as ncm_linear_bf16. Device pointers. */
int ncm_linear_bf16_residual(ncm_ctx_t* ctx, const uint16_t* x, const uint16_t* w,
                             const uint16_t* bias, const float* residual, void* y,
                             int64_t m, int64_t k, int64_t n, int out_mode);

/* The projection and the SwiGLU that follows it in the decoder's MLP
 * (src/decoder.zig:206-211, bf16 mode) in one pass: y[m, j] =
 * round(silu_bf16(gate[m, j]) * up[m, j]) with gate and up the bf16 outputs
 * of the gate and up projections. w: bf16 [n2, k] holding the gate and up
 * rows interleaved in groups of 32 (rows 64g .. 64g+31 = gate rows
 * 32g .. 32g+31, rows 64g+32 .. 64g+63 = up rows 32g .. 32g+31; bias, if
 * given, in the same order); n2 = 2 * intermediate, a multiple of 64.
 * y: uint16 bf16 bits [m, n2 / 2]. The same bits as ncm_linear_bf16 (BF16)
 * followed by ncm_silu_mul_dev. Device pointers; y 8-byte aligned. */
int ncm_linear_bf16_swiglu(ncm_ctx_t* ctx, const uint16_t* x, const uint16_t* w,
                           const uint16_t* bias, uint16_t* y, int64_t m, int64_t k,
                           int64_t n2);

/* The q|k|v projection and the RoPE rotation of its q and k heads
 * (root.zig:497-530) in one pass, for head_dim 64: y = the bf16 output of
 * ncm_linear_bf16 (BF16), with every 64-wide head in columns [0, rot_cols)
 * rotated as ncm_rope_rotate_dev does (table row = row % seq_len). n and
 * rot_cols multiples of 64. The same bits as the two calls in sequence.
 * Device pointers; y 8-byte aligned. */
int ncm_linear_bf16_rope64(ncm_ctx_t* ctx, const uint16_t* x, const uint16_t* w,
                           const uint16_t* bias, uint16_t* y, int64_t m, int64_t k, int64_t n,
                           int64_t rot_cols, int64_t seq_len, const float* cosine,
                           const float* sine);

/* y[m, n] = sum_k x[m, k] * w[n, k], fp32 operands and accumulation on the
 * fp32 MFMA (device counterpart of packages/kernels/root.zig:25-65).
 * Requires k % 4 == 0 and 16-byte aligned x and w. Device pointers. */
int ncm_linear_f32(ncm_ctx_t* ctx, const float* x, const float* w, float* y, int64_t m,
                   int64_t k, int64_t n);

/* f32 -> bf16 bits, RNE, NaN -> 0x7FC0 (packages/bf16/root.zig:17-22).
 * flush != 0 additionally flushes subnormal results to signed zero (the
 * operand treatment of root.zig:124-135). Device pointers. */
int ncm_bf16_from_f32_dev(ncm_ctx_t* ctx, const float* src, uint16_t* dst, int64_t n,
                          int flush);
/* bf16 bits -> f32, exact (packages/bf16/root.zig:25-37). Device pointers. */
int ncm_bf16_widen_dev(ncm_ctx_t* ctx, const uint16_t* src, float* dst, int64_t n);

/* Device RMSNorm of each of `rows` rows of x [rows, width] (f32) with weight
 * [width] (f32): the decoder's normalize_rows (src/decoder.zig:168), one row
 * per wavefront. out_mode NCM_OUT_BF16_F32 (y float) or NCM_OUT_BF16 (y
 * uint16 bits, ready for ncm_linear_bf16): the bf16 mode (rms_norm_bf16,
 * root.zig:246-254), same bits as ncm_rms_norm_bf16; NCM_OUT_F32 (y float):
 * the f32 mode (rms_norm, root.zig:226-239), same bits as the reference. y
 * may be x. When width % 4 == 0, x and weight must be 16-byte aligned. */
int ncm_rms_norm_rows_dev(ncm_ctx_t* ctx, const float* x, const float* weight, void* y,
                          int64_t rows, int64_t width, float epsilon, int out_mode);

/* Device MLP activation (src/decoder.zig:210-211). out_mode NCM_OUT_BF16_F32
 * or NCM_OUT_BF16: bf16 mode, y[i] = round_bf16(silu_bf16(gate[i]) * up[i]);
 * NCM_OUT_F32: f32 mode, y[i] = silu(gate[i]) * up[i] (root.zig:255-261).
 * up NULL gives the SiLU alone; y may be gate. */
int ncm_silu_mul_dev(ncm_ctx_t* ctx, const float* gate, const float* up, void* y, int64_t n,
                     int out_mode);

/* Device RoPE rotation, bf16 mode: rotate_head (packages/kernels/root.zig:
 * 615-634) applied in place to every head of every row, as attention_impl
 * does for queries and keys (root.zig:497-530). x: uint16 bf16 bits, row r
 * holds `heads` heads of head_dim values at x[r * row_stride + h * head_dim];
 * row r rotates by table row r % seq_len of cosine/sine (float
 * [seq_len, head_dim], the rope_tables layout, root.zig:328-348). Table
 * entries, products and sums are rounded to bf16 in the reference's order:
 * bit-identical to the reference. Device pointers. */
int ncm_rope_rotate_dev(ncm_ctx_t* ctx, uint16_t* x, int64_t rows, int64_t row_stride,
                        int heads, int head_dim, int64_t seq_len, const float* cosine,
                        const float* sine);

/* Device causal attention, bf16 mode: the scores, softmax and context of
 * attention_impl (root.zig:536-578) with the causal_mask of the decoder
 * (root.zig:380-399, src/decoder.zig:155) for `batch` sequences of seq_len
 * tokens each (positions 0 .. seq_len - 1; window 0 = no sliding window).
 * q: uint16 bits [batch * seq_len, q_stride] (head h at column h * head_dim);
 * k, v: uint16 bits [batch * seq_len, kv_stride]; query head h reads key/value
 * head h / (q_heads / kv_heads). out: [batch * seq_len, out_stride], float
 * holding bf16 values (NCM_OUT_BF16_F32) or uint16 bits (NCM_OUT_BF16,
 * ready for the output projection). head_dim 64 or 128; strides multiples of
 * 8 elements; q, k, v 16-byte aligned. Scores and P V are summed on the MFMA
 * in its own order (the reference sums in key order), so results agree with
 * the reference within a few bf16 steps rather than bit for bit. */
int ncm_attention_bf16_dev(ncm_ctx_t* ctx, const uint16_t* q, const uint16_t* k,
                           const uint16_t* v, void* out, int64_t batch, int64_t seq_len,
                           int q_heads, int kv_heads, int head_dim, int64_t q_stride,
                           int64_t kv_stride, int64_t out_stride, int64_t window, int out_mode);

/* The same attention under NCM's block-diagonal level mask
 * (src/ncm_mask.zig:10-42) instead of the causal one: key k is allowed for
 * query q when k is an unpadded prefix key (k < prefix_len) or lies in q's
 * level block [seg_lo[q], seg_hi[q]) (prefix queries: an empty block).
 * seg_lo, seg_hi: device int32 [seq_len] (positions within one sequence,
 * the same for every sequence of the batch), from
 * ncm_block_diagonal_segments; prefix_pad_bits: device uint64
 * [ceil(prefix_len / 64)] (bit k % 64 of word k / 64 = prefix key k padded)
 * or NULL. A query with no allowed key gets a zero context (root.zig:563-565).
 * Other arguments and the tolerance as ncm_attention_bf16_dev. */
int ncm_attention_bf16_seg_dev(ncm_ctx_t* ctx, const uint16_t* q, const uint16_t* k,
                               const uint16_t* v, void* out, int64_t batch, int64_t seq_len,
                               int q_heads, int kv_heads, int head_dim, int64_t q_stride,
                               int64_t kv_stride, int64_t out_stride, int64_t prefix_len,
                               const int32_t* seg_lo, const int32_t* seg_hi,
                               const uint64_t* prefix_pad_bits, int out_mode);

/* Host: the block-diagonal mask of block_diagonal_mask (src/ncm_mask.zig:
 * 10-42) in the compact form the attention reads: per position the level
 * block [seg_lo, seg_hi) (empty for the prefix) and the prefix pad flags
 * packed into bits (pad_bits [ceil(prefix_len / 64)], may be NULL).
 * NCM_E_LENGTH where the reference returns InvalidPrefixMask (pad_len not 0
 * or prefix_len) or InvalidMaskSize (prefix + levels != seq_len). */
int ncm_block_diagonal_segments(int64_t prefix_len, const int64_t* level_lengths,
                                int64_t n_levels, const uint8_t* prefix_pad_mask,
                                int64_t pad_len, int64_t seq_len, int32_t* seg_lo,
                                int32_t* seg_hi, uint64_t* pad_bits);

/* Codebook-tied code head of the NCM generator (described at PROJECT.md:222,
 * upstream _TiedCodebookHead; the reference has no code for it yet):
 *   logits[r, k] = (2 z_r . E_k - csq[k]) * scale (+ bias[k]),
 *   scale = expf(log_inv_t) / d_scale, d_scale = mean_k csq[k]
 * with z: bf16 [rows, d] (the head's projection of the hidden state), E: the
 * level's bf16 codebook [v, d], csq: fp32 [v] = ||E_k||^2 (ncm_rvq_prepare),
 * bias: fp32 [v] or NULL, logits: fp32 [rows, v]. The bf16 MFMA of the RVQ
 * distance with the affine map in its epilogue; d_scale is summed in f64 on
 * the device. argmax_k logits[r] is the nearest code to z_r. d % 8 == 0,
 * z and E 16-byte aligned, v >= 1. Device pointers. */
int ncm_tied_head_logits(ncm_ctx_t* ctx, const uint16_t* z, const uint16_t* codebook,
                         const float* csq, const float* bias, float log_inv_t, float* logits,
                         int64_t rows, int64_t d, int64_t v);

/* Every level's tied head of the level-parallel step in one launch: z holds
 * the levels' rows one level after another (level_rows[l] rows of level l,
 * host array), codebooks: bf16 [n_levels, v, d], csq: fp32 [n_levels, v],
 * bias: fp32 [n_levels, v] or NULL, log_inv_t: host float [n_levels] (one
 * learned scalar per level's head), logits: fp32 [sum rows, v]. Level l's
 * rows get level l's codebook, norms, bias and scale; each as
 * ncm_tied_head_logits. 1 <= n_levels <= 32. */
int ncm_tied_head_logits_levels(ncm_ctx_t* ctx, const uint16_t* z, const uint16_t* codebooks,
                                const float* csq, const float* bias, const float* log_inv_t,
                                const int64_t* level_rows, int64_t n_levels, int64_t d,
                                int64_t v, float* logits);

/* ---- bf16 decoder prefill forward (src/decoder.zig:62-228) ---- */

/* Model shape (config.spec_t fields the forward reads). window: sliding
 * window, 0 = none. */
typedef struct ncm_decoder_shape {
    int64_t hidden;        /* hidden_size */
    int64_t intermediate;  /* intermediate_size */
    int64_t vocab;         /* vocab_size */
    int32_t q_heads;       /* num_attention_heads */
    int32_t kv_heads;      /* num_key_value_heads */
    int32_t head_dim;      /* 64 or 128 */
    int32_t layers;        /* num_hidden_layers */
    int64_t window;        /* sliding_window, 0 = none */
    float rms_eps;         /* rms_norm_eps */
} ncm_decoder_shape_t;

/* One layer's device weights (bf16 bits unless stated). The projections the
 * reference keeps separate (attention_weights_t, root.zig:351-362; the MLP
 * weights of decoder.zig) are row-concatenated: qkv_weight holds the q rows
 * [q_heads * head_dim], then the k rows, then the v rows [kv_heads *
 * head_dim each], each row `hidden` wide; gate_up_weight holds the gate and
 * up rows interleaved in groups of 32 as ncm_linear_bf16_swiglu reads them
 * (intermediate % 32 == 0). Biases follow the same row order; NULL = no
 * bias. */
typedef struct ncm_decoder_layer {
    const float* input_norm;           /* [hidden] */
    const uint16_t* qkv_weight;        /* [(q_heads + 2 kv_heads) head_dim, hidden] */
    const uint16_t* qkv_bias;          /* [(q_heads + 2 kv_heads) head_dim] or NULL */
    const uint16_t* o_weight;          /* [hidden, q_heads head_dim] */
    const uint16_t* o_bias;            /* [hidden] or NULL */
    const float* post_attention_norm;  /* [hidden] */
    const uint16_t* gate_up_weight;    /* [2 intermediate, hidden], interleaved */
    const uint16_t* gate_up_bias;      /* [2 intermediate] or NULL, interleaved */
    const uint16_t* down_weight;       /* [hidden, intermediate] */
    const uint16_t* down_bias;         /* [hidden] or NULL */
    /* QK-norm scales (Qwen3, root.zig:501-530): rms_norm_bf16 of every q and
     * k head before the rotation; both NULL or both float [head_dim]. */
    const float* q_norm;
    const float* k_norm;
    /* Norm biases (rms_norm_rows_with_bias, src/ncm_norm.zig:22-49): float
     * [hidden] added (and rounded to bf16) after the norm, or NULL. */
    const float* input_norm_bias;
    const float* post_attention_norm_bias;
} ncm_decoder_layer_t;

/* Bf16 prefill forward of `batch` sequences of seq_len tokens each (the
 * reference's forward, decoder.zig:62-228 with bf16_compute, applied to each
 * sequence; positions restart at 0 in every sequence). token_ids: HOST int64
 * [batch * seq_len], each < vocab (else NCM_E_ARG, the reference's
 * TokenIdOutOfRange). layers: HOST array [shape->layers] of device weight
 * pointers. embed: bf16 [vocab, hidden]; lm_head: bf16 [vocab, hidden] or
 * NULL for tied embeddings; final_norm: float [hidden]; cosine, sine: float
 * [seq_len, head_dim] RoPE tables (rope_tables layout, root.zig:328-348,
 * built on the host with the system libm as the reference does). logits:
 * float [batch * seq_len, vocab] (bf16 values, token-major). Intermediates
 * live in the context's workspace. A layer with q_norm / k_norm applies the
 * QK-norm (Qwen3 layouts). Linear outputs, scores and P V are summed in MFMA
 * order, so logits agree with the reference within bf16 tolerance, not bit
 * for bit. trace: NULL or the stages of forward_with_trace to keep
 * (decoder_trace_t, src/decoder.zig:30-47; ncm_decoder_trace_t below), as
 * float holding the bf16 values; the projections the fused kernels never
 * store (attention_output, gate_projection, up_projection, mlp_output) are
 * computed again for the trace with the same sums. */
typedef struct ncm_decoder_trace ncm_decoder_trace_t;
int ncm_decoder_forward_dev(ncm_ctx_t* ctx, const ncm_decoder_shape_t* shape,
                            const ncm_decoder_layer_t* layers, const uint16_t* embed,
                            const float* final_norm, const uint16_t* lm_head,
                            const float* cosine, const float* sine, const int64_t* token_ids,
                            int64_t batch, int64_t seq_len, float* logits,
                            const ncm_decoder_trace_t* trace);

/* One layer's device weights in the f32 mode (decoder.zig:10-20,
 * attention_weights_t of root.zig:351-362), all float: qkv_weight holds the
 * q rows [q_heads * head_dim], then the k rows, then the v rows [kv_heads *
 * head_dim each], each `hidden` wide (q|k|v biases in the same order);
 * gate, up and down as stored ([intermediate, hidden], [intermediate,
 * hidden], [hidden, intermediate]). NULL = no bias; q_norm / k_norm: both
 * NULL or both [head_dim]. */
typedef struct ncm_decoder_layer_f32 {
    const float* input_norm;           /* [hidden] */
    const float* qkv_weight;           /* [(q_heads + 2 kv_heads) head_dim, hidden] */
    const float* qkv_bias;             /* [(q_heads + 2 kv_heads) head_dim] or NULL */
    const float* o_weight;             /* [hidden, q_heads head_dim] */
    const float* o_bias;               /* [hidden] or NULL */
    const float* post_attention_norm;  /* [hidden] */
    const float* gate_weight;          /* [intermediate, hidden] */
    const float* gate_bias;            /* [intermediate] or NULL */
    const float* up_weight;            /* [intermediate, hidden] */
    const float* up_bias;              /* [intermediate] or NULL */
    const float* down_weight;          /* [hidden, intermediate] */
    const float* down_bias;            /* [hidden] or NULL */
    const float* q_norm;               /* [head_dim] or NULL */
    const float* k_norm;               /* [head_dim] or NULL */
    /* rms_norm_rows_with_bias (src/ncm_norm.zig:22-49): biases added after
     * the input and post-attention norms, or NULL (the decoder has none). */
    const float* input_norm_bias;      /* [hidden] or NULL */
    const float* post_attention_norm_bias; /* [hidden] or NULL */
} ncm_decoder_layer_f32_t;

/* The per-stage trace of forward_with_trace (decoder_trace_t,
 * src/decoder.zig:30-47): device float buffers, each NULL (not kept) or
 * [layers, batch * seq_len, width] layer-major (block_input: [batch *
 * seq_len, hidden]); width is hidden, q_heads * head_dim (attention_context)
 * or intermediate (gate_projection, up_projection, gate_up_product). */
struct ncm_decoder_trace {
    float* block_input;
    float* input_norm;
    float* attention_context;
    float* attention_output;
    float* attention_residual;
    float* post_attention_norm;
    float* gate_projection;
    float* up_projection;
    float* gate_up_product;
    float* mlp_output;
    float* block_output;
};

/* The prefill forward in the reference's f32 mode (forward_with_trace with
 * bf16_compute false, decoder.zig:62-228: rms_norm, kernels.matmul + bias,
 * f32 rotate_head and attention, silu, unrounded adds), for `batch`
 * sequences of seq_len tokens. Arguments as ncm_decoder_forward_dev with
 * float weights (embed and lm_head float [vocab, hidden], lm_head NULL for
 * tied embeddings); trace: NULL or the stages to keep. hidden,
 * intermediate and head_dim must be multiples of 4 (head_dim <= 256) and
 * q_heads * head_dim too; logits: float [batch * seq_len, vocab]. The
 * projections sum on the fp32 MFMA in its own order; the attention sums in
 * the reference's dimension and key order; exp is the device's. */
int ncm_decoder_forward_f32_dev(ncm_ctx_t* ctx, const ncm_decoder_shape_t* shape,
                                const ncm_decoder_layer_f32_t* layers, const float* embed,
                                const float* final_norm, const float* lm_head,
                                const float* cosine, const float* sine,
                                const int64_t* token_ids, int64_t batch, int64_t seq_len,
                                float* logits, const ncm_decoder_trace_t* trace);

/* ---- NCM level-parallel body (src/ncm_model.zig) ---- */

#define NCM_MAX_LEVELS 32

/* Attention pattern of the NCM body. */
enum {
    NCM_MASK_BLOCK_DIAGONAL = 0, /* the reference's block_diagonal_mask
                                    (src/ncm_mask.zig:10-42, decision D8):
                                    prefix keys (unpadded) and the own level */
    NCM_MASK_BLOCK_CAUSAL = 1,   /* unpadded prefix keys and every level up to
                                    and including the query's own */
    NCM_MASK_CAUSAL = 2          /* config.source_causal: causal over the
                                    sequence, optional sliding window */
};

/* config_t (src/ncm_model.zig:15-35) without the RoPE fields (the tables
 * come precomputed) and with the mask choice. */
typedef struct ncm_ncm_shape {
    int64_t hidden;         /* hidden_size, % 8 == 0 */
    int64_t vq_width;       /* vq_width, % 8 == 0 */
    int64_t intermediate;   /* intermediate_size, % 32 == 0 */
    int32_t q_heads;        /* num_attention_heads */
    int32_t kv_heads;       /* num_key_value_heads */
    int32_t head_dim;       /* 64 or 128 */
    int32_t layers;         /* >= 1 */
    int64_t prefix_length;
    int64_t prefix_vocab;   /* rows of prefix_token_embedding */
    int32_t n_levels;       /* 1 .. NCM_MAX_LEVELS */
    int32_t mask_mode;      /* NCM_MASK_* */
    int32_t query_level0;   /* nonzero: l0_queries replace level 0's inputs */
    int32_t use_level_encoding; /* nonzero: add level_embedding */
    int64_t window;         /* sliding window of NCM_MASK_CAUSAL, 0 = none */
    float rms_eps;          /* rms_norm_epsilon */
    int32_t reserved;       /* 0 */
    int64_t level_lengths[NCM_MAX_LEVELS];
} ncm_ncm_shape_t;

/* weights_t (src/ncm_model.zig:61-72) on the device, bf16 bits unless
 * stated. conv_weight / conv_bias: HOST arrays [n_levels] of device float
 * pointers ([vq_width, vq_width, 3] in the reference's [out][in][tap] order,
 * and [vq_width]) for post_upsample_convs, or both NULL for none. */
typedef struct ncm_ncm_weights {
    const uint16_t* prefix_token_embedding; /* [prefix_vocab, vq_width] */
    const uint16_t* input_projection;       /* [hidden, vq_width] */
    const uint16_t* input_projection_bias;  /* [hidden] */
    const uint16_t* level_embedding;        /* [n_levels, hidden] */
    const uint16_t* l0_queries;             /* [level_lengths[0], vq_width] or NULL */
    const float* final_norm;                /* [hidden] */
    const float* final_norm_bias;           /* [hidden] or NULL */
    const float* const* conv_weight;
    const float* const* conv_bias;
} ncm_ncm_weights_t;

/* The NCM body forward (forward_with_trace, src/ncm_model.zig:89-250) for
 * one prefix and one target sequence, in the
 * bf16 mode of the source decoder: bf16 projections with fp32 accumulation
 * (operands rounded and flushed as matmul_bf16 does), rms_norm_bf16,
 * silu_bf16, bf16 attention, every add rounded to bf16; the convolutions
 * run in fp32. prefix_ids: HOST int64 [prefix_length], each < prefix_vocab
 * (else NCM_E_ARG, PrefixTokenOutOfRange). prefix_pad_mask: HOST uint8
 * [pad_len], pad_len 0 or prefix_length (else NCM_E_LENGTH,
 * InvalidPrefixMask). target_inputs: float [sum level_lengths, vq_width].
 * layers: HOST array [layers] (ncm_decoder_layer_t: fused q|k|v rows, gate
 * and up rows interleaved in groups of 32, optional QK-norm and norm biases
 * as ln_1_bias / ln_2_bias). cosine, sine: float [S, head_dim], S =
 * prefix_length + sum level_lengths, the RoPE tables gathered at the
 * positions of fill_level_positions (src/ncm_position.zig:11-118).
 * output: float [S, hidden] (bf16 values), the final-normalized hidden
 * states in [prefix | levels] order. hidden_states: NULL or float
 * [layers + 1, S, hidden], the reference's trace (ncm_model.zig:169-171,
 * :243-249): the input stage, the output of layers 0 .. layers - 2, then the
 * final-normalized states. Intermediates live in the context's
 * workspace. */
int ncm_ncm_forward_dev(ncm_ctx_t* ctx, const ncm_ncm_shape_t* shape,
                        const ncm_decoder_layer_t* layers, const ncm_ncm_weights_t* weights,
                        const int64_t* prefix_ids, const uint8_t* prefix_pad_mask,
                        int64_t pad_len, const float* target_inputs, const float* cosine,
                        const float* sine, float* output, float* hidden_states);

/* weights_t (src/ncm_model.zig:61-72) for the f32 body: every tensor float.
 * conv_weight / conv_bias as in ncm_ncm_weights_t. */
typedef struct ncm_ncm_weights_f32 {
    const float* prefix_token_embedding; /* [prefix_vocab, vq_width] */
    const float* input_projection;       /* [hidden, vq_width] */
    const float* input_projection_bias;  /* [hidden] or NULL */
    const float* level_embedding;        /* [n_levels, hidden] */
    const float* l0_queries;             /* [level_lengths[0], vq_width] or NULL */
    const float* final_norm;             /* [hidden] */
    const float* final_norm_bias;        /* [hidden] or NULL */
    const float* const* conv_weight;
    const float* const* conv_bias;
} ncm_ncm_weights_f32_t;

/* The NCM body forward in the reference's own arithmetic: f32 throughout
 * (kernels.matmul + bias, src/ncm_model.zig:278-294; rms_norm_rows_with_bias;
 * f32 RoPE at the restarting positions; f32 attention with the level mask,
 * each dot product in dimension order and the softmax sum and context in
 * key order; silu(gate) * up; unrounded adds). Arguments, checks and output
 * layout as ncm_ncm_forward_dev, with float weights and
 * ncm_decoder_layer_f32_t layers (fused q|k|v rows, gate / up / down as
 * stored, norm biases as input_norm_bias / post_attention_norm_bias).
 * hidden, vq_width, intermediate and head_dim must be multiples of 4,
 * head_dim <= 256. The projections sum on the fp32 MFMA in its own order,
 * so results agree with the reference to fp32 rounding, not bit for bit. */
int ncm_ncm_forward_f32_dev(ncm_ctx_t* ctx, const ncm_ncm_shape_t* shape,
                            const ncm_decoder_layer_f32_t* layers,
                            const ncm_ncm_weights_f32_t* weights, const int64_t* prefix_ids,
                            const uint8_t* prefix_pad_mask, int64_t pad_len,
                            const float* target_inputs, const float* cosine, const float* sine,
                            float* output, float* hidden_states);

/* ---- multiscale residual vector quantization ---- */

/* csq[l * v + k] = squared norm of codebook row (l, k), in the fixed fp32
 * order of the oracle (64 strided lanes, halving tree). Device pointers. */
int ncm_rvq_prepare(ncm_ctx_t* ctx, const uint16_t* codebooks, int64_t levels, int64_t v,
                    int64_t d, float* csq);

/* Multiscale RVQ encode. x: float [b, t, d]; strides: host int32 [levels],
 * powers of two, non-increasing, t % strides[0] == 0 (level l pools by
 * strides[l] and repeats back); codebooks: bf16 [levels, v, d]; csq from
 * ncm_rvq_prepare. Outputs (device): codes int32 [b, sum_l t/s_l] (level 0
 * first); recon float [b, t, d] or NULL (sum of the selected code vectors);
 * gap float (codes layout) or NULL: relative gap between the two smallest
 * full distances among the exactly rescored candidates (+inf when only one
 * candidate needed rescoring). force_codes (device, codes layout) or NULL:
 * teacher forcing; when given, later levels' residuals are built from these
 * codes while `codes` still receives this library's own argmin.
 * Requires d % 64 == 0, d <= 4096 (NCM_E_SHAPE above: the row kernels hold
 * a row in registers), v <= 65536. n_flagged (host, nullable) receives the
 * number of rows for which some group of codes had more near-best members
 * than the approximate pass kept, so that every code of the group was
 * rescored exactly (a synchronizing read). */
int ncm_rvq_encode(ncm_ctx_t* ctx, const float* x, int64_t b, int64_t t, int64_t d,
                   int64_t levels, const int32_t* strides, const uint16_t* codebooks,
                   const float* csq, int64_t v, int32_t* codes, float* recon, float* gap,
                   const int32_t* force_codes, int64_t* n_flagged);

/* ncm_rvq_encode that also reports, per level, how the exact pass went. No
 * counterpart in the reference (which has no RVQ code); for callers that
 * profile or tune the encode. flagged and scored (host, int64 [levels])
 * receive the rows with an incomplete candidate chunk (every code of the
 * chunk rescored) and the rows that needed any exact distance (every other
 * row had exactly one candidate under its error bound, which is then the
 * exact argmin without a rescore). Synchronizes the context's stream. */
int ncm_rvq_encode_counts(ncm_ctx_t* ctx, const float* x, int64_t b, int64_t t, int64_t d,
                          int64_t levels, const int32_t* strides, const uint16_t* codebooks,
                          const float* csq, int64_t v, int32_t* codes, float* recon, float* gap,
                          const int32_t* force_codes, int64_t* flagged, int64_t* scored);

/* Allocation-free variant of ncm_rvq_encode. No counterpart in the
 * reference: it exists for callers that cannot allocate device memory (code
 * under HIP graph capture, serving loops, harnesses that forbid hipMalloc).
 * Same arguments, results and stream ordering as ncm_rvq_encode without
 * n_flagged. Its workspace is a fixed device array of NCM_RVQ_SCRATCH_BYTES
 * per GPU, held until the process ends; a shape that needs more returns
 * NCM_E_SCRATCH (ncm_last_error() gives both sizes) before any device work.
 * It calls no hipMalloc / hipFree. Calls on one GPU share that array and are
 * ordered through one event per device (created by ncm_init): a call on any
 * stream or host thread runs after the previous call's kernels. On a stream
 * under graph capture that event is left out, and the caller orders captured
 * calls that share a GPU. */
#define NCM_RVQ_SCRATCH_BYTES (64u << 20)
int ncm_rvq_encode_noalloc(ncm_ctx_t* ctx, const float* x, int64_t b, int64_t t, int64_t d,
                           int64_t levels, const int32_t* strides, const uint16_t* codebooks,
                           const float* csq, int64_t v, int32_t* codes, float* recon,
                           float* gap, const int32_t* force_codes);

/* recon[b, t, :] = sum over levels (in order) of codebooks[l][codes_l]. */
int ncm_rvq_decode(ncm_ctx_t* ctx, const int32_t* codes, int64_t b, int64_t t, int64_t d,
                   int64_t levels, const int32_t* strides, const uint16_t* codebooks,
                   int64_t v, float* recon);

/* ---- safetensors weights (packages/safetensors/root.zig) ---- */

/* Reader for the safetensors header and the sharded index, with the
 * reference's checks in its order (root.zig:148-193, 197-228): the 8-byte
 * little-endian length (>= 8 bytes, <= 100 000 000), valid UTF-8, a JSON
 * object of tensors {"dtype", "shape", "data_offsets"} and an optional
 * "__metadata__" of strings, known dtypes, offsets contiguous from 0 in
 * data-offset order, shape and bit products without overflow, whole bytes,
 * sizes matching shapes, file = prefix + header + data. Malformed input
 * returns NCM_E_FORMAT with the reference's error name in ncm_last_error()
 * ("HeaderTooSmall", "HeaderTooLarge", "InvalidHeaderLength", "InvalidUtf8",
 * "InvalidHeader", "UnknownDtype", "InvalidOffsets", "ShapeOverflow",
 * "MisalignedBits", "SizeMismatch", "FileSizeMismatch", "InvalidIndex",
 * "UnsafeShardName"; "SyntaxError" for JSON that does not parse). */
#define NCM_ST_MAX_DIMS 8
typedef struct ncm_st_file ncm_st_file_t;
typedef struct ncm_st_index ncm_st_index_t;
typedef struct ncm_st_tensor {
    const char* name;        /* owned by the file handle; a name that holds
                                U+0000 reads as cut there, and ncm_st_find
                                does not match it (ncm_st_tensor still
                                lists it) */
    int32_t dtype;           /* index in the reference's Dtype order: BOOL 0, U8, I8,
                                U16, I16, U32, I32, U64, I64, F4, F6_E2M3, F6_E3M2,
                                F8_E5M2, F8_E4M3, F8_E8M0, F8_E4M3FNUZ, F8_E5M2FNUZ,
                                F16 17, BF16 18, F32 19, F64 20, C64 21 */
    int32_t ndim;
    uint64_t shape[NCM_ST_MAX_DIMS];
    uint64_t data_begin;     /* byte range inside the data section */
    uint64_t data_end;
} ncm_st_tensor_t;

/* Parses a header held in memory: bytes starts with the 8-byte prefix and
 * holds at least the JSON header; file_size is the whole file's size
 * (parse_header, root.zig:148-193). */
int ncm_st_parse(const void* bytes, size_t len, uint64_t file_size, ncm_st_file_t** out);
/* Maps a .safetensors file and parses its header. */
int ncm_st_open(const char* path, ncm_st_file_t** out);
int ncm_st_close(ncm_st_file_t* f);
int ncm_st_summary(const ncm_st_file_t* f, uint64_t* header_len, uint64_t* data_len,
                   int64_t* tensor_count);
/* Tensor i in data-offset order; NCM_E_SHAPE (info filled, shape cut) when
 * ndim > NCM_ST_MAX_DIMS. */
int ncm_st_tensor(const ncm_st_file_t* f, int64_t index, ncm_st_tensor_t* out);
int ncm_st_find(const ncm_st_file_t* f, const char* name, ncm_st_tensor_t* out);
const char* ncm_st_dtype_name(int dtype);
int ncm_st_dtype_bits(int dtype);
/* Copies a tensor's stored bytes to device memory (dst_bytes must equal its
 * size) on the context's stream through the context's two pinned staging
 * buffers (up to 64 MiB each, allocated by the first upload that needs them
 * and kept until ncm_destroy); the bytes are on the device when the call
 * returns. bf16 weights reach the device as stored, without the loader's
 * widen to f32 (src/loader.zig:339-342). The file must come from
 * ncm_st_open. */
int ncm_st_upload(ncm_ctx_t* ctx, const ncm_st_file_t* f, const char* name, void* dst,
                  size_t dst_bytes);
/* Sharded index (model.safetensors.index.json, parse_index, root.zig:197-228):
 * weight_map of tensor -> plain shard file name, optional metadata.total_size. */
int ncm_st_parse_index(const char* json, size_t len, ncm_st_index_t** out);
int ncm_st_index_close(ncm_st_index_t* ix);
int64_t ncm_st_index_count(const ncm_st_index_t* ix);
int ncm_st_index_entry(const ncm_st_index_t* ix, int64_t i, const char** tensor,
                       const char** shard);
/* NCM_E_ARG when the index has no metadata.total_size. */
int ncm_st_index_total_size(const ncm_st_index_t* ix, uint64_t* total);

/* ------------------------------------------------------------------------
 * The upstream VQ-VAE tokenizer (inference): encoder, multiscale residual
 * quantizer and decoder of research/reference/vq_forward_semantics.md, in
 * the configuration of the released WMT14 tokenizer
 * (research/converter/wmt14_tokenizer_keys.md) or any other of that module.
 * The reference has no code for it (ROADMAP.md:259-261 plans a Zig port,
 * packages/vq); these entry points follow the conventions of the kernels
 * module (caller-owned device buffers, explicit sizes, int status).
 * Float32 arithmetic throughout, in the device's summation order.
 * ------------------------------------------------------------------------ */
#define NCM_VQ_TOK_MAX_LEVELS 64
#define NCM_VQ_TOK_MAX_STAGES 8

/* Shapes, switches and device weights of one tokenizer. Conv weights are
 * packed by ncm_vq_tok_pack_conv_dev from their PyTorch layouts. */
typedef struct ncm_vq_tok {
    int64_t embed_dim;       /* D: a multiple of 4 * groups */
    int64_t in_vocab;        /* C: token table rows */
    int64_t context_length;  /* wpe rows, >= the sequence length */
    int32_t n_levels;        /* K, 1 .. NCM_VQ_TOK_MAX_LEVELS */
    int32_t groups;          /* GroupNorm groups of the pre-quant and cascade norms */
    /* Positions of each level, increasing; the last one is the sequence
     * length L (the levels of vq.levels, models/quant.py:285-292). */
    int64_t level_len[NCM_VQ_TOK_MAX_LEVELS];
    int64_t level_vocab[NCM_VQ_TOK_MAX_LEVELS];  /* V_l: codebook rows */
    float group_eps;         /* GroupNorm epsilon (1e-5) */
    float resi_ratio;        /* Phi blend ratio r (0.5) */
    /* Level 0 through the learned conv cascade (learned_l1_sampling with
     * learned_l1_cascade): n_stages kernel = stride = stage_stride[i] convs
     * whose strides multiply to L / level_len[0]; GroupNorm after every
     * inner down stage and up stage (cascade_norm) and after the last down
     * stage (cascade_norm_final). 0: level 0 pools by area and upsamples
     * linearly like the other levels. */
    int32_t learned_level0;
    int32_t n_stages;
    int64_t stage_stride[NCM_VQ_TOK_MAX_STAGES];
    int32_t cascade_norm;
    int32_t cascade_norm_final;
    /* Device weights (float32, 16-byte aligned). */
    const float* wte;                                 /* [C, D] (encode only) */
    const float* wpe;                                 /* [context_length, D] */
    const float* codebook[NCM_VQ_TOK_MAX_LEVELS];     /* [V_l, D] */
    /* Phi of each level (quant_resi.l): Conv1d(D, D, 3, padding 1) packed
     * [D, 3 D] and its bias [D]; weight NULL: no Phi (Q = the upsampled
     * codes). */
    const float* resi_weight[NCM_VQ_TOK_MAX_LEVELS];
    const float* resi_bias[NCM_VQ_TOK_MAX_LEVELS];
    const float* down_weight[NCM_VQ_TOK_MAX_STAGES];  /* packed [D, s D] */
    const float* down_bias[NCM_VQ_TOK_MAX_STAGES];    /* [D] */
    const float* up_weight[NCM_VQ_TOK_MAX_STAGES];    /* packed [s D, D] */
    const float* up_bias[NCM_VQ_TOK_MAX_STAGES];      /* [D] */
} ncm_vq_tok_t;

/* Repacks a conv weight for ncm_vq_tok_t: transposed 0 takes a Conv1d
 * weight (out = c, in = c, k) to dst[o, j c + i] = src[o, i, j] ([c, k c]);
 * transposed 1 a ConvTranspose1d weight (in = c, out = c, k) to
 * dst[j c + o, i] = src[i, o, j] ([k c, c]). Device buffers of c c k floats. */
int ncm_vq_tok_pack_conv_dev(ncm_ctx_t* ctx, const float* src, float* dst, int64_t c, int64_t k,
                             int transposed);

/* Tokenizer encode in eval mode for `batch` sequences of L = level_len[K-1]
 * token ids (host int64 [batch, L], each in [0, C): NCM_E_ARG otherwise,
 * before any device work): z = GroupNorm(wte[ids] + wpe) (the encoder and
 * pre-quant norm, vq_forward_semantics.md:38-49), then the quantizer loop
 * (models/quant.py:448-549, vq_forward_semantics.md:59-76): per level l,
 * u = Down_l(r), codes = argmin_k |u - e_k|^2 (lowest index on ties), Q =
 * Phi_l(Up_l(e[codes])), zhat += Q, r -= Q. codes: int32 [batch, sum_l
 * level_len[l]], level 0 first; zhat (NULL: not kept) and latent (z, NULL:
 * not kept): float [batch, L, D]. The search computes |e|^2 - 2 u.e on the
 * fp32 MFMA, so a code may differ from PyTorch's where two distances agree
 * to float32 rounding. */
int ncm_vq_tok_encode_dev(ncm_ctx_t* ctx, const ncm_vq_tok_t* tok, const int64_t* token_ids,
                          int64_t batch, int32_t* codes, float* zhat, float* latent);

/* The quantizer alone from a latent z (device float [batch, L, D]). */
int ncm_vq_tok_quantize_dev(ncm_ctx_t* ctx, const ncm_vq_tok_t* tok, const float* latent,
                            int64_t batch, int32_t* codes, float* zhat);

/* zhat = sum_l Phi_l(Up_l(e_l[codes_l])) (the decoder's input in eval mode);
 * codes as ncm_vq_tok_encode_dev writes them. A code outside [0, V_l) is
 * clamped into it (the lookup stays in bounds; this stream-ordered entry
 * cannot report it), so a caller validates caller-made codes first, as
 * upstream's embedding lookup would raise (the Python mirror refuses them
 * with NCM_E_ARG before the call). */
int ncm_vq_tok_reconstruct_dev(ncm_ctx_t* ctx, const ncm_vq_tok_t* tok, const int32_t* codes,
                               int64_t batch, float* zhat);

/* The tokenizer's decoder (models/vae.py:198-258 in eval mode,
 * vq_forward_semantics.md:84-94): x = zhat; x += c_proj(attn(LN_1(x)));
 * x += mlp.c_proj(GELU(mlp.c_fc(LN_2(x)))); logits = output_layer(ln_f(x)).
 * Attention is bidirectional over the L positions, n_head heads of D /
 * n_head, with q and k RMS-normalised per head when q_norm / k_norm are set
 * (both or neither). Device float32 weights in PyTorch's Linear layout [out,
 * in]; LayerNorm biases may be NULL (ln_f has none). */
typedef struct ncm_vq_tok_decoder {
    int32_t n_head;
    float ln_eps;                /* LayerNorm epsilon (1e-6) */
    float qk_eps;                /* q / k RMSNorm epsilon (1e-6) */
    const float* ln1_weight;     /* [D] */
    const float* ln1_bias;       /* [D] or NULL */
    const float* attn_weight;    /* c_attn [3 D, D]: q, k, v rows */
    const float* attn_bias;      /* [3 D] or NULL */
    const float* proj_weight;    /* attn.c_proj [D, D] */
    const float* proj_bias;      /* [D] or NULL */
    const float* q_norm;         /* [D / n_head] or NULL */
    const float* k_norm;         /* [D / n_head] or NULL */
    const float* ln2_weight;     /* [D] */
    const float* ln2_bias;       /* [D] or NULL */
    const float* fc_weight;      /* mlp.c_fc [4 D, D] */
    const float* fc_bias;        /* [4 D] or NULL */
    const float* fc_proj_weight; /* mlp.c_proj [D, 4 D] */
    const float* fc_proj_bias;   /* [D] or NULL */
    const float* lnf_weight;     /* ln_f [D] (no bias) */
    const float* out_weight;     /* output_layer [C, D] (no bias) */
} ncm_vq_tok_decoder_t;

/* logits (float [batch, L, C], C = tok->in_vocab) of the decoder on zhat
 * (float [batch, L, D], as ncm_vq_tok_encode_dev or
 * ncm_vq_tok_reconstruct_dev write it). Only the shapes of tok are read. */
int ncm_vq_tok_decode_dev(ncm_ctx_t* ctx, const ncm_vq_tok_t* tok,
                          const ncm_vq_tok_decoder_t* dec, const float* zhat, int64_t batch,
                          float* logits);

#ifdef __cplusplus
}
#endif

#endif /* NCMORPH_AMD_H */
