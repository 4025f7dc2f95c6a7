// Host-side launchers of the HIP kernels (internal to the library).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace ncm {

// Tile configuration chosen for an M x N output (see the table in
// linear.hip); a valid `forced` index overrides the choice.
int linear_tile_config(int64_t M, int64_t N, int64_t K, int forced);

hipError_t launch_linear(const uint16_t* x, const uint16_t* w, const uint16_t* bias, void* y,
                         int64_t M, int64_t K, int64_t N, int out_mode, int config,
                         hipStream_t stream);
// The reference's matmul_bf16 arithmetic bit for bit (VALU pair-order fma
// chains, 512 / 1024 K blocks, operand and partial flush): x [M, K], w
// [N, K] bf16 with row stride K, bias bf16 [N] or null, y [M, N].
hipError_t launch_linear_exact(const uint16_t* x, const uint16_t* w, const uint16_t* bias,
                               void* y, int64_t M, int64_t K, int64_t N, int out_mode,
                               hipStream_t stream);

// y = residual + linear (bf16 modes: round_bf16(residual + round_bf16(linear)));
// residual fp32 [M, N], may equal y for the fp32 output mode.
hipError_t launch_linear_residual(const uint16_t* x, const uint16_t* w, const uint16_t* bias,
                                  const float* residual, void* y, int64_t M, int64_t K,
                                  int64_t N, int out_mode, hipStream_t stream);

// Linear + SwiGLU (bf16 bits out, y [M, N2 / 2]); w rows interleaved in
// groups of 32 (gate, up); N2 % 64 == 0. See linear_fused.hip.
hipError_t launch_linear_swiglu(const uint16_t* x, const uint16_t* w, const uint16_t* bias,
                                uint16_t* y, int64_t M, int64_t K, int64_t N2,
                                hipStream_t stream);
// Linear + bf16 RoPE of 64-wide heads in columns [0, rot_cols) (bf16 bits out,
// y [M, N]); N and rot_cols multiples of 64.
hipError_t launch_linear_rope64(const uint16_t* x, const uint16_t* w, const uint16_t* bias,
                                uint16_t* y, int64_t M, int64_t K, int64_t N, int64_t rot_cols,
                                int64_t seq_len, const float* cosine, const float* sine,
                                hipStream_t stream);

// Rows past the last full 256-row tile that launch_linear,
// launch_linear_residual and launch_linear_swiglu (automatic tile choice)
// hand to linear_tail.hip, or 0: M % 256 when it is at most 64, the
// 256 x 256 tile is chosen for M and for M - M % 256, K % 2048 == 0,
// N % 16 == 0, and the partial row tile would cost the whole chip an extra
// round (N: the weight's rows).
int64_t linear_tail_rows(int64_t M, int64_t N, int64_t K);
// The R rows of such a tail (x, y, residual pointing at its first row):
// out_mode / bias / residual as launch_linear(_residual); swiglu: N is the
// feature count (weight rows 2 N, interleaved as launch_linear_swiglu),
// y [R, N] bf16 bits.
hipError_t launch_linear_tail(const uint16_t* x, const uint16_t* w, const uint16_t* bias,
                              const float* residual, void* y, int64_t R, int64_t K, int64_t N,
                              int out_mode, bool swiglu, hipStream_t st);

// fp32 operands, fp32 output; K % 4 == 0, 16-byte aligned x and w.
hipError_t launch_linear_f32(const float* x, const float* w, float* y, int64_t M, int64_t K,
                             int64_t N, hipStream_t stream);

// RMSNorm (bf16 mode, pinned cascade) of `rows` rows of width n; out_mode
// NCM_OUT_BF16_F32 (f32 holding bf16 values) or NCM_OUT_BF16 (bits).
hipError_t launch_rms_norm_rows(const float* x, const float* weight, void* y, int64_t rows,
                                int64_t n, float epsilon, int out_mode, hipStream_t stream);
// QK-norm (rms_norm_bf16 per head, in place on bf16 bits; hd <= 256).
hipError_t launch_qk_norm(uint16_t* x, int64_t rows, int64_t row_stride, int heads, int hd,
                          const float* weight, float epsilon, hipStream_t stream);
// y = round_bf16(y + bias[column]) in place over [rows, n] (bits: bf16 bits,
// else floats holding bf16 values).
hipError_t launch_bias_round(void* y, const float* bias, int64_t rows, int64_t n, bool bits,
                             hipStream_t stream);
// y = round_bf16(silu_bf16(gate) * up) (up NULL: silu_bf16(gate) alone).
hipError_t launch_silu_mul(const float* gate, const float* up, void* y, int64_t n, int out_mode,
                           hipStream_t stream);

// RoPE rotate-half (bf16 mode) in place on bf16 bits; see decoder_ops.hip.
// Codebook-tied head logits of `levels` levels in one launch: level l's rows
// (rows[l] of them, after those of the levels before it) against codebook l:
// y = (2 z E_l^T - csq_l) * expf(log_inv_t[l]) / mean(csq_l) (+ bias_l);
// scale: `levels` floats of device scratch. log_inv_t and rows: host arrays.
hipError_t launch_tied_head(const uint16_t* z, const uint16_t* cb, const float* csq,
                            const float* bias, const float* log_inv_t, const int64_t* rows,
                            int levels, float* scale, float* y, int64_t d, int64_t v,
                            hipStream_t st);
hipError_t launch_rope_rotate(uint16_t* x, int64_t rows, int64_t row_stride, int heads, int hd,
                              int64_t seq_len, const float* cosine, const float* sine,
                              hipStream_t stream);
// Causal (optionally windowed) bf16 attention over `batch` sequences of
// seq_len tokens; see attention.hip. vt: device scratch of
// attention_workspace_bytes(batch, seq_len, kv_heads, head_dim) bytes,
// 16-byte aligned (the transposed V).
size_t attention_workspace_bytes(int64_t batch, int64_t seq_len, int kv_heads, int head_dim);
hipError_t launch_attention_bf16(const uint16_t* q, const uint16_t* k, const uint16_t* v,
                                 void* out, int64_t batch, int64_t seq_len, int q_heads,
                                 int kv_heads, int head_dim, int64_t q_stride, int64_t kv_stride,
                                 int64_t out_stride, int64_t window, int out_mode, uint16_t* vt,
                                 hipStream_t stream);

// The same attention with the prefix + level-block mask (see attention.hip).
hipError_t launch_attention_bf16_seg(const uint16_t* q, const uint16_t* k, const uint16_t* v,
                                     void* out, int64_t batch, int64_t seq_len, int q_heads,
                                     int kv_heads, int head_dim, int64_t q_stride,
                                     int64_t kv_stride, int64_t out_stride, int64_t prefix,
                                     const int32_t* seg_lo, const int32_t* seg_hi,
                                     const uint64_t* pad, int out_mode, uint16_t* vt,
                                     hipStream_t stream);

hipError_t launch_bf16_from_f32(const float* src, uint16_t* dst, int64_t n, int flush,
                                hipStream_t stream);
// Row-padded variant: src [rows, cols] -> dst [rows, ld] (ld >= cols),
// columns [cols, ld) zero-filled.
hipError_t launch_bf16_from_f32_2d(const float* src, uint16_t* dst, int64_t rows, int64_t cols,
                                   int64_t ld, int flush, hipStream_t stream);
hipError_t launch_bf16_widen(const uint16_t* src, float* dst, int64_t n, hipStream_t stream);

}  // namespace ncm
