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
    size_t o_hidden, o_normed, o_qkv, o_ctx, o_act, o_ids, o_vt, o_gu, total;
};

Plan plan(const ncm_decoder_shape_t& s, int64_t batch, int64_t seq,
          const ncm_decoder_trace_t* trace) {
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
    p.o_gu = off;     off += up(trace_gu_bytes(s, p.T, trace));
    p.total = off;
    return p;
}

}  // namespace

size_t decoder_workspace_bytes(const ncm_decoder_shape_t& s, int64_t batch, int64_t seq,
                               const ncm_decoder_trace_t* trace) {
    return plan(s, batch, seq, trace).total;
}

size_t trace_gu_bytes(const ncm_decoder_shape_t& s, int64_t T, const ncm_decoder_trace_t* trace) {
    if (!trace || (!trace->gate_projection && !trace->up_projection)) return 0;
    return (size_t)T * 2 * s.intermediate * 2;
}

// gate[r, f] and up[r, f] (widened) of the gate|up projection gu [T, 2 I]
// whose rows are interleaved in groups of 32 (gate features 32 p .. 32 p + 31
// at columns 64 p .. 64 p + 31, up features at 64 p + 32 .. 64 p + 63);
// either output may be null.
__global__ __launch_bounds__(256) void gate_up_split_kernel(const uint16_t* __restrict__ gu,
                                                            int64_t T, int64_t I,
                                                            float* __restrict__ gate,
                                                            float* __restrict__ up) {
    const int64_t n = T * I;
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n;
         i += (int64_t)gridDim.x * 256) {
        const int64_t r = i / I, f = i - r * I;
        const uint16_t* row = gu + r * 2 * I + 64 * (f / 32) + f % 32;
        if (gate) gate[i] = __uint_as_float((uint32_t)row[0] << 16);
        if (up) up[i] = __uint_as_float((uint32_t)row[32] << 16);
    }
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
    const ncm_decoder_trace_t* tr = a.trace;
    // Trace copies: bf16 bits widened, fp32 rows copied.
    auto widen = [&](float* base, int64_t l, const uint16_t* src, int64_t width) -> hipError_t {
        if (!base) return hipSuccess;
        return launch_bf16_widen(src, base + l * T * width, T * width, st);
    };
    auto copy = [&](float* base, int64_t l) -> hipError_t {
        if (!base) return hipSuccess;
        return hipMemcpyAsync(base + l * T * H, a.hidden, (size_t)T * H * 4,
                              hipMemcpyDeviceToDevice, st);
    };
    for (int l = 0; l < s.layers; ++l) {
        const ncm_decoder_layer_t& L = a.layers[l];
        NCM_TRY(launch_rms_norm_rows(a.hidden, L.input_norm, a.normed, T, H, s.rms_eps,
                                     NCM_OUT_BF16, st));
        if (L.input_norm_bias)
            NCM_TRY(launch_bias_round(a.normed, L.input_norm_bias, T, H, true, st));
        if (tr) NCM_TRY(widen(tr->input_norm, l, a.normed, H));
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
        if (tr) {
            NCM_TRY(widen(tr->attention_context, l, a.ctx, q_w));
            // The o projection alone (the fused residual launch below computes
            // the same sums for the hidden update).
            if (tr->attention_output)
                NCM_TRY(launch_linear(a.ctx, L.o_weight, L.o_bias, tr->attention_output + l * T * H,
                                      T, q_w, H, NCM_OUT_BF16_F32, -1, st));
        }
        NCM_TRY(launch_linear_residual(a.ctx, L.o_weight, L.o_bias, a.hidden, a.hidden, T, q_w, H,
                                       NCM_OUT_BF16_F32, st));
        if (tr) NCM_TRY(copy(tr->attention_residual, l));
        NCM_TRY(launch_rms_norm_rows(a.hidden, L.post_attention_norm, a.normed, T, H, s.rms_eps,
                                     NCM_OUT_BF16, st));
        if (L.post_attention_norm_bias)
            NCM_TRY(launch_bias_round(a.normed, L.post_attention_norm_bias, T, H, true, st));
        if (tr) {
            NCM_TRY(widen(tr->post_attention_norm, l, a.normed, H));
            if (tr->gate_projection || tr->up_projection) {
                // The gate|up projection without the SwiGLU epilogue, then split.
                NCM_TRY(launch_linear(a.normed, L.gate_up_weight, L.gate_up_bias, a.trace_gu, T, H,
                                      2 * I, NCM_OUT_BF16, -1, st));
                const int64_t blocks = (T * I + 255) / 256 < 4096 ? (T * I + 255) / 256 : 4096;
                hipLaunchKernelGGL(gate_up_split_kernel, dim3((unsigned)blocks), dim3(256), 0, st,
                                   a.trace_gu, T, I,
                                   tr->gate_projection ? tr->gate_projection + l * T * I : nullptr,
                                   tr->up_projection ? tr->up_projection + l * T * I : nullptr);
                NCM_TRY(hipGetLastError());
            }
        }
        NCM_TRY(launch_linear_swiglu(a.normed, L.gate_up_weight, L.gate_up_bias, a.act, T, H,
                                     2 * I, st));
        if (tr) {
            NCM_TRY(widen(tr->gate_up_product, l, a.act, I));
            if (tr->mlp_output)
                NCM_TRY(launch_linear(a.act, L.down_weight, L.down_bias, tr->mlp_output + l * T * H,
                                      T, I, H, NCM_OUT_BF16_F32, -1, st));
        }
        NCM_TRY(launch_linear_residual(a.act, L.down_weight, L.down_bias, a.hidden, a.hidden, T,
                                       I, H, NCM_OUT_BF16_F32, st));
        if (tr) NCM_TRY(copy(tr->block_output, l));
    }
    return hipSuccess;
}

hipError_t decoder_forward(const ncm_decoder_shape_t& s, const ncm_decoder_layer_t* layers,
                           const uint16_t* embed, const float* final_norm,
                           const uint16_t* lm_head, const float* cosine, const float* sine,
                           const int64_t* host_ids, int64_t batch, int64_t seq, float* logits,
                           const ncm_decoder_trace_t* trace, void* ws, hipStream_t st) {
    const Plan p = plan(s, batch, seq, trace);
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
    a.trace = trace;
    a.trace_gu = (uint16_t*)(w + p.o_gu);
    int64_t* ids = (int64_t*)(w + p.o_ids);
    const int64_t T = p.T, H = s.hidden;

    NCM_TRY(hipMemcpyAsync(ids, host_ids, (size_t)T * 8, hipMemcpyHostToDevice, st));
    {
        const unsigned gx = (unsigned)((H + 511) / 512 < 8 ? (H + 511) / 512 : 8);
        hipLaunchKernelGGL(embed_rows_kernel, dim3(gx, (unsigned)T), dim3(256), 0, st, ids, embed,
                           a.hidden, H);
        NCM_TRY(hipGetLastError());
    }
    if (trace && trace->block_input)
        NCM_TRY(hipMemcpyAsync(trace->block_input, a.hidden, (size_t)T * H * 4,
                               hipMemcpyDeviceToDevice, st));
    NCM_TRY(run_layers(a, st));
    NCM_TRY(launch_rms_norm_rows(a.hidden, final_norm, a.normed, T, H, s.rms_eps, NCM_OUT_BF16,
                                 st));
    return launch_linear(a.normed, lm_head ? lm_head : embed, nullptr, logits, T, H, s.vocab,
                         NCM_OUT_BF16_F32, -1, st);
}

}  // namespace ncm
