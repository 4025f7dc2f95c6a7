// Decoder prefill forward (internal; the C entry point is in api.hip).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/ncmorph_amd.h"

namespace ncm {

size_t decoder_workspace_bytes(const ncm_decoder_shape_t& s, int64_t batch, int64_t seq,
                               const ncm_decoder_trace_t* trace = nullptr);

// The layer stack of the bf16 forward over `batch` sequences of `seq` rows:
// hidden [batch * seq, hidden] fp32 (bf16 values) is updated in place.
// Attention: causal with shape->window, or, when seg_lo is set, the prefix +
// level-block mask of ncm_attention_bf16_seg_dev. cosine / sine: [seq,
// head_dim], table row = row % seq. Scratch: normed [rows, hidden], qkv
// [rows, (q_heads + 2 kv_heads) head_dim], ctx [rows, q_heads head_dim], act
// [rows, intermediate], all bf16 bits.
struct LayerStack {
    const ncm_decoder_shape_t* shape;
    const ncm_decoder_layer_t* layers;  // host array [shape->layers]
    int64_t batch, seq;
    const float* cosine;
    const float* sine;
    int64_t prefix;
    const int32_t* seg_lo;
    const int32_t* seg_hi;
    const uint64_t* pad;
    float* hidden;
    uint16_t* normed;
    uint16_t* qkv;
    uint16_t* ctx;
    uint16_t* act;
    uint16_t* vt;  // attention_workspace_bytes(batch, seq, kv_heads, head_dim)
    // Nullable: the stages of decoder_trace_t to keep, each [layers, T,
    // width] (block_input is not written here). trace_gu: bf16 [T, 2 I]
    // scratch for the unfused gate|up projection, needed when the gate or
    // up projection is traced.
    const ncm_decoder_trace_t* trace;
    uint16_t* trace_gu;
};
hipError_t run_layers(const LayerStack& a, hipStream_t st);
// Bytes of trace_gu for T rows (0 when the trace keeps neither projection).
size_t trace_gu_bytes(const ncm_decoder_shape_t& s, int64_t T, const ncm_decoder_trace_t* trace);

// All pointers device memory except `layers` (host array) and `host_ids`.
hipError_t decoder_forward(const ncm_decoder_shape_t& s, const ncm_decoder_layer_t* layers,
                           const uint16_t* embed, const float* final_norm,
                           const uint16_t* lm_head, const float* cosine, const float* sine,
                           const int64_t* host_ids, int64_t batch, int64_t seq, float* logits,
                           const ncm_decoder_trace_t* trace, void* ws, hipStream_t st);

// f32 mode (decoder_f32.hip): workspace bytes and the forward. All pointers
// device memory except `layers` (host array) and `host_ids`; trace may be
// null.
size_t decoder_f32_workspace_bytes(const ncm_decoder_shape_t& s, int64_t batch, int64_t seq);
hipError_t decoder_forward_f32(const ncm_decoder_shape_t& s, const ncm_decoder_layer_f32_t* layers,
                               const float* embed, const float* final_norm, const float* lm_head,
                               const float* cosine, const float* sine, const int64_t* host_ids,
                               int64_t batch, int64_t seq, float* logits,
                               const ncm_decoder_trace_t* trace, void* ws, hipStream_t st);

// The f32 layer stack (decoder_f32.hip) over `batch` sequences of `seq`
// rows: hidden [batch * seq, hidden] fp32 updated in place. Attention:
// causal with shape->window, or, when seg_lo is set, the prefix + level-block
// mask (prefix keys without their pad bit, then keys [seg_lo, seg_hi) of the
// query's row). cosine / sine: [seq, head_dim], table row = row % seq.
// Scratch (fp32): normed [rows, hidden], q [rows, q_heads head_dim], k, v
// [rows, kv_heads head_dim], ctx [rows, q_heads head_dim], proj [rows,
// hidden], gate, up [rows, intermediate]. trace may be null.
struct LayerStackF32 {
    const ncm_decoder_shape_t* shape;
    const ncm_decoder_layer_f32_t* layers;  // host array [shape->layers]
    int64_t batch, seq;
    const float* cosine;
    const float* sine;
    int64_t prefix;
    const int32_t* seg_lo;
    const int32_t* seg_hi;
    const uint64_t* pad;
    float *hidden, *normed, *q, *k, *v, *ctx, *proj, *gate, *up;
    const ncm_decoder_trace_t* trace;
};
hipError_t run_layers_f32(const LayerStackF32& a, hipStream_t st);

// y [rows, n] = x [rows, k] w^T (+ bias) on the fp32 MFMA (k % 4 == 0).
hipError_t project_f32(const float* x, const float* w, const float* bias, float* y, int64_t rows,
                       int64_t k, int64_t n, hipStream_t st);
// y[r, c] += a[r, c] (a_rows == rows) or a[c] (a_rows == 1).
hipError_t launch_add_f32(float* y, const float* a, int64_t rows, int64_t n, int64_t a_rows,
                          hipStream_t st);

}  // namespace ncm
