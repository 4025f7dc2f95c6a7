// The bf16 decoder prefill forward of src/decoder.zig:62-228 on one GPU:
// stream-ordered launches of the linear, RMSNorm, RoPE, attention and MLP
// kernels over a batch of equal-length sequences, with every intermediate
// resident in the context's workspace. Per layer (bf16 mode):
//   n   = rms_norm_bf16(h, input_norm)                 -> bf16 bits
//   qkv = n W_qkv^T (+ b), q and k heads rotated       -> bf16 bits, one GEMM
//         (RoPE table row = position in the sequence; fused for head_dim 64)
//   c   = attention(q, k, v)                           -> bf16 bits
//   h   = round(h + round(c W_o^T (+ b)))              (fused residual)
//   n   = rms_norm_bf16(h, post_attention_norm)
//   a   = round(silu_bf16(n W_gate^T) * n W_up^T)      -> bf16 bits, one GEMM
//         over the interleaved gate/up rows with the SwiGLU in its epilogue
//   h   = round(h + round(a W_down^T (+ b)))           (fused residual)
// then logits = round(rms_norm_bf16(h, final_norm) W_head^T). With q_norm /
// k_norm the q and k heads take rms_norm_bf16 before the rotation (QK-norm,
// root.zig:501-530); norm biases are added after their norm and rounded.
// run_layers is the layer stack alone, shared with the NCM body, whose
// attention takes the level mask instead of the causal one.
// The reference runs q, k and v (and gate and up) as separate projections of
// the same input; one GEMM over the row-concatenated weights computes each
// output column by the same dot product.
#include <hip/hip_runtime.h>

#include "common.h"
#include "decoder.h"
#include "linear.h"

namespace ncm {

// hidden[r] = widened embed[ids[r]] (bf16 -> f32 is exact, so the
// reference's round_bf16 of the embedding rows is the identity here).
__global__ __launch_bounds__(256) void embed_rows_kernel(const int64_t* __restrict__ ids,
                                                         const uint16_t* __restrict__ table,
                                                         float* __restrict__ hidden,
                                                         int64_t width) {
    const int64_t r = blockIdx.y;
    const uint16_t* src = table + ids[r] * width;
    float* dst = hidden + r * width;
    for (int64_t i = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 2; i < width;
         i += (int64_t)gridDim.x * 512) {
        if (i + 1 < width) {
            const uint32_t p = *(const uint32_t*)(src + i);
            dst[i] = __uint_as_float(p << 16);
            dst[i + 1] = __uint_as_float(p & 0xFFFF0000u);
        } else {
            dst[i] = __uint_as_float((uint32_t)src[i] << 16);
        }
    }
}

namespace {

constexpr size_t kAlign = 256;
size_t up(size_t n) { return (n + kAlign - 1) / kAlign * kAlign; }

struct Plan {
    int64_t T, qkv_w, q_w;
    size_t o_hidden, o_normed, o_qkv, o_ctx, o_act, o_ids, o_vt, total;
};

Plan plan(const ncm_decoder_shape_t& s, int64_t batch, int64_t seq) {
    Plan p;
    p.T = batch * seq;
    p.q_w = (int64_t)s.q_heads * s.head_dim;
    p.qkv_w = (int64_t)(s.q_heads + 2 * s.kv_heads) * s.head_dim;
    size_t off = 0;
    p.o_hidden = off; off += up((size_t)p.T * s.hidden * 4);
    p.o_normed = off; off += up((size_t)p.T * s.hidden * 2);
    p.o_qkv = off;    off += up((size_t)p.T * p.qkv_w * 2);
    p.o_ctx = off;    off += up((size_t)p.T * p.q_w * 2);
    p.o_act = off;    off += up((size_t)p.T * s.intermediate * 2);
    p.o_ids = off;    off += up((size_t)p.T * 8);
    p.o_vt = off;     off += up(attention_workspace_bytes(batch, seq, s.kv_heads, s.head_dim));
    p.total = off;
    return p;
}

}  // namespace

size_t decoder_workspace_bytes(const ncm_decoder_shape_t& s, int64_t batch, int64_t seq) {
    return plan(s, batch, seq).total;
}

#define NCM_TRY(call)                                  \
    do {                                               \
        hipError_t e_ = (call);                        \
        if (e_ != hipSuccess) return e_;               \
    } while (0)

hipError_t run_layers(const LayerStack& a, hipStream_t st) {
    const ncm_decoder_shape_t& s = *a.shape;
    const int64_t T = a.batch * a.seq, H = s.hidden, I = s.intermediate;
    const int hd = s.head_dim;
    const int64_t q_w = (int64_t)s.q_heads * hd;
    const int64_t qkv_w = (int64_t)(s.q_heads + 2 * s.kv_heads) * hd;
    for (int l = 0; l < s.layers; ++l) {
        const ncm_decoder_layer_t& L = a.layers[l];
        NCM_TRY(launch_rms_norm_rows(a.hidden, L.input_norm, a.normed, T, H, s.rms_eps,
                                     NCM_OUT_BF16, st));
        if (L.input_norm_bias)
            NCM_TRY(launch_bias_round(a.normed, L.input_norm_bias, T, H, true, st));
        if (hd == 64 && !L.q_norm) {  // rotation fused into the projection's epilogue
            NCM_TRY(launch_linear_rope64(a.normed, L.qkv_weight, L.qkv_bias, a.qkv, T, H, qkv_w,
                                         (int64_t)(s.q_heads + s.kv_heads) * hd, a.seq, a.cosine,
                                         a.sine, st));
        } else {
            NCM_TRY(launch_linear(a.normed, L.qkv_weight, L.qkv_bias, a.qkv, T, H, qkv_w,
                                  NCM_OUT_BF16, -1, st));
            if (L.q_norm) {  // QK-norm precedes the rotation (root.zig:501-530)
                NCM_TRY(launch_qk_norm(a.qkv, T, qkv_w, s.q_heads, hd, L.q_norm, s.rms_eps, st));
                NCM_TRY(launch_qk_norm(a.qkv + q_w, T, qkv_w, s.kv_heads, hd, L.k_norm, s.rms_eps,
                                       st));
            }
            NCM_TRY(launch_rope_rotate(a.qkv, T, qkv_w, s.q_heads, hd, a.seq, a.cosine, a.sine,
                                       st));
            NCM_TRY(launch_rope_rotate(a.qkv + q_w, T, qkv_w, s.kv_heads, hd, a.seq, a.cosine,
                                       a.sine, st));
        }
        const uint16_t* kp = a.qkv + q_w;
        const uint16_t* vp = kp + (int64_t)s.kv_heads * hd;
        if (a.seg_lo)
            NCM_TRY(launch_attention_bf16_seg(a.qkv, kp, vp, a.ctx, a.batch, a.seq, s.q_heads,
                                              s.kv_heads, hd, qkv_w, qkv_w, q_w, a.prefix,
                                              a.seg_lo, a.seg_hi, a.pad, NCM_OUT_BF16, a.vt,
                                              st));
        else
            NCM_TRY(launch_attention_bf16(a.qkv, kp, vp, a.ctx, a.batch, a.seq, s.q_heads,
                                          s.kv_heads, hd, qkv_w, qkv_w, q_w, s.window,
                                          NCM_OUT_BF16, a.vt, st));
        NCM_TRY(launch_linear_residual(a.ctx, L.o_weight, L.o_bias, a.hidden, a.hidden, T, q_w, H,
                                       NCM_OUT_BF16_F32, st));
        NCM_TRY(launch_rms_norm_rows(a.hidden, L.post_attention_norm, a.normed, T, H, s.rms_eps,
                                     NCM_OUT_BF16, st));
        if (L.post_attention_norm_bias)
            NCM_TRY(launch_bias_round(a.normed, L.post_attention_norm_bias, T, H, true, st));
        NCM_TRY(launch_linear_swiglu(a.normed, L.gate_up_weight, L.gate_up_bias, a.act, T, H,
                                     2 * I, st));
        NCM_TRY(launch_linear_residual(a.act, L.down_weight, L.down_bias, a.hidden, a.hidden, T,
                                       I, H, NCM_OUT_BF16_F32, st));
    }
    return hipSuccess;
}

hipError_t decoder_forward(const ncm_decoder_shape_t& s, const ncm_decoder_layer_t* layers,
                           const uint16_t* embed, const float* final_norm,
                           const uint16_t* lm_head, const float* cosine, const float* sine,
                           const int64_t* host_ids, int64_t batch, int64_t seq, float* logits,
                           void* ws, hipStream_t st) {
    const Plan p = plan(s, batch, seq);
    char* w = (char*)ws;
    LayerStack a{};
    a.shape = &s;
    a.layers = layers;
    a.batch = batch;
    a.seq = seq;
    a.cosine = cosine;
    a.sine = sine;
    a.hidden = (float*)(w + p.o_hidden);
    a.normed = (uint16_t*)(w + p.o_normed);
    a.qkv = (uint16_t*)(w + p.o_qkv);
    a.ctx = (uint16_t*)(w + p.o_ctx);
    a.act = (uint16_t*)(w + p.o_act);
    a.vt = (uint16_t*)(w + p.o_vt);
    int64_t* ids = (int64_t*)(w + p.o_ids);
    const int64_t T = p.T, H = s.hidden;

    NCM_TRY(hipMemcpyAsync(ids, host_ids, (size_t)T * 8, hipMemcpyHostToDevice, st));
    {
        const unsigned gx = (unsigned)((H + 511) / 512 < 8 ? (H + 511) / 512 : 8);
        hipLaunchKernelGGL(embed_rows_kernel, dim3(gx, (unsigned)T), dim3(256), 0, st, ids, embed,
                           a.hidden, H);
        NCM_TRY(hipGetLastError());
    }
    NCM_TRY(run_layers(a, st));
    NCM_TRY(launch_rms_norm_rows(a.hidden, final_norm, a.normed, T, H, s.rms_eps, NCM_OUT_BF16,
                                 st));
    return launch_linear(a.normed, lm_head ? lm_head : embed, nullptr, logits, T, H, s.vocab,
                         NCM_OUT_BF16_F32, -1, st);
}

}  // namespace ncm
