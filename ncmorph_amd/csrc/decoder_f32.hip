// The decoder prefill forward of src/decoder.zig:62-228 in its f32 mode
// (bf16_compute false: checkpoints that are not all BF16), with the
// per-stage trace of forward_with_trace. Per layer, all in fp32:
//   n    = rms_norm(h, input_norm)                          (root.zig:226-239)
//   q, k, v = n W^T (+ b)  -> [QK-norm] -> rotate_head      (root.zig:483-530, 615-634)
//   c    = softmax((q . k) / sqrt(hd) over allowed keys) v   (root.zig:536-578)
//   h    = h + (c W_o^T (+ b))
//   n    = rms_norm(h, post_attention_norm)
//   a    = silu(n W_gate^T (+ b)) * (n W_up^T (+ b))         (root.zig:255-261)
//   h    = h + (a W_down^T (+ b))
// then logits = rms_norm(h, final_norm) W_head^T. The projections run on the
// fp32 MFMA (launch_linear_f32: every product exact, the sums in the matrix
// core's order instead of the reference's increasing k); the bias is added
// after the product, as the reference's project does. The attention sums
// each dot product in dimension order, the softmax sum and every context
// element in key order, as the reference, so only exp differs (device expf
// against Zig's exp).
#include <hip/hip_runtime.h>

#include "common.h"
#include "decoder.h"
#include "linear.h"

namespace ncm {

namespace {

// hidden[r] = embed[ids[r]] (f32 table rows).
__global__ __launch_bounds__(256) void embed_rows_f32_kernel(const int64_t* __restrict__ ids,
                                                             const float* __restrict__ table,
                                                             float* __restrict__ hidden,
                                                             int64_t width) {
    const int64_t r = blockIdx.y;
    const float* src = table + ids[r] * width;
    float* dst = hidden + r * width;
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < width;
         i += (int64_t)gridDim.x * 256)
        dst[i] = src[i];
}

// y[r, c] = y[r, c] + a[r, c] (a_rows = rows) or + a[c] (a_rows = 1, a bias).
__global__ __launch_bounds__(256) void add_f32_kernel(float* __restrict__ y,
                                                      const float* __restrict__ a, int64_t rows,
                                                      int64_t n, int64_t a_rows) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= rows * n) return;
    const float av = a_rows == 1 ? a[i % n] : a[i];
    y[i] = y[i] + av;
}

// rotate_head in f32 mode (root.zig:615-634), in place: row r, head h at
// x[r * row_stride + h * hd ..]; table row r % seq_len. One thread per pair.
__global__ __launch_bounds__(256) void rope_rotate_f32_kernel(float* __restrict__ x, int64_t rows,
                                                              int64_t row_stride, int heads,
                                                              int hd, int64_t seq_len,
                                                              const float* __restrict__ cosine,
                                                              const float* __restrict__ sine) {
    const int half = hd >> 1;
    const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= rows * heads * half) return;
    const int i = (int)(idx % half);
    const int64_t rh = idx / half;
    const int h = (int)(rh % heads);
    const int64_t r = rh / heads;
    const int64_t pos = r % seq_len;
    float* e = x + r * row_stride + (int64_t)h * hd + i;
    const float first = e[0], second = e[half];
    const float* ct = cosine + pos * hd + i;
    const float* st = sine + pos * hd + i;
    const float left = first * ct[0];
    const float right = -second * st[0];
    const float right2 = first * st[half];
    const float left2 = second * ct[half];
    e[0] = left + right;
    e[half] = left2 + right2;
}

hipError_t launch_rope_rotate_f32(float* x, int64_t rows, int64_t row_stride, int heads, int hd,
                                  int64_t seq_len, const float* cosine, const float* sine,
                                  hipStream_t st) {
    const int64_t n = rows * heads * (hd / 2);
    if (n == 0) return hipSuccess;
    hipLaunchKernelGGL(rope_rotate_f32_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0,
                       st, x, rows, row_stride, heads, hd, seq_len, cosine, sine);
    return hipGetLastError();
}

constexpr int kAttnF32MaxHd = 256;

// f32-mode attention of one (sequence, query, head) per wavefront, four
// heads per workgroup: grid (seq_len, ceil(q_heads / 4), batch). Allowed
// keys, in increasing order: causal, [k_lo, query] (optionally windowed); or
// with the level mask (seg_lo set), the prefix keys 0 .. prefix-1 whose pad
// bit is clear, then [seg_lo[q], seg_hi[q]) (at or after the prefix). They
// are walked 64 per chunk, one per lane, three times: the maximum score; the
// softmax sum, added in key order (every lane adds the chunk's exponentials
// in lane order); then p = exp(s - max) / sum and the context, lane =
// dimension, adding p_k v_k in key order. A score is the dot product in
// dimension order, then times 1 / sqrt(hd). Masked keys (probability 0) add
// nothing, as in the reference unless V holds an infinity or NaN there; a
// query with no allowed key gets a zero context (root.zig:563-565).
__global__ __launch_bounds__(256) void attention_f32_kernel(
    const float* __restrict__ q, const float* __restrict__ k, const float* __restrict__ v,
    float* __restrict__ out, int64_t T, int q_heads, int group, int hd, int64_t q_stride,
    int64_t kv_stride, int64_t out_stride, int64_t window, float scale, int64_t prefix,
    const int32_t* __restrict__ seg_lo, const int32_t* __restrict__ seg_hi,
    const uint64_t* __restrict__ pad) {
    const int lane = threadIdx.x & 63;
    const int h = blockIdx.y * 4 + (threadIdx.x >> 6);
    if (h >= q_heads) return;
    const int64_t b = blockIdx.z, qi = blockIdx.x;
    const int kvh = h / group;
    const float* qrow = q + (b * T + qi) * q_stride + (int64_t)h * hd;
    const float* kbase = k + b * T * kv_stride + (int64_t)kvh * hd;
    const float* vbase = v + b * T * kv_stride + (int64_t)kvh * hd;
    // q spread over the lanes: dimension d in lane d % 64, slot d / 64.
    float qv[kAttnF32MaxHd / 64];
#pragma unroll
    for (int s = 0; s < kAttnF32MaxHd / 64; ++s) {
        const int d = s * 64 + lane;
        qv[s] = d < hd ? qrow[d] : 0.0f;
    }
    // Key j of the walk (j in [0, nkeys)) and whether it is allowed.
    int64_t nkeys, k_lo = 0, lo = 0, P = 0;
    if (seg_lo) {
        P = prefix;
        lo = seg_lo[b * T + qi];
        const int64_t hi = seg_hi[b * T + qi];
        nkeys = P + (hi > lo ? hi - lo : 0);
    } else {
        k_lo = window > 0 ? qi - window + 1 : 0;
        if (k_lo < 0) k_lo = 0;
        nkeys = qi + 1 - k_lo;
    }
    auto key_of = [&](int64_t j) { return seg_lo ? (j < P ? j : lo + (j - P)) : k_lo + j; };
    auto allowed = [&](int64_t j) {
        if (j >= nkeys) return false;
        if (seg_lo && j < P && pad) return ((pad[j >> 6] >> (j & 63)) & 1ull) == 0ull;
        return true;
    };
    // q . k in dimension order (separate multiply and add), then * scale;
    // the q values come from their lanes, the k row in 16-byte loads.
    auto score_of = [&](int64_t key) {
        const float* kr = kbase + key * kv_stride;
        float s = 0.0f;
#pragma unroll
        for (int sl = 0; sl < kAttnF32MaxHd / 64; ++sl) {
            if (sl * 64 >= hd) break;
            const uint32_t qbits = __float_as_uint(qv[sl]);
            const int nd = hd - sl * 64 < 64 ? hd - sl * 64 : 64;
            for (int j = 0; j < nd; j += 4) {
                const f32x4_t k4 = *(const f32x4_t*)(kr + sl * 64 + j);
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    s = s + __uint_as_float(__builtin_amdgcn_readlane(qbits, j + e)) * k4[e];
            }
        }
        return s * scale;
    };
    // Walk 1: the maximum.
    float m = -INFINITY;
    for (int64_t c0 = 0; c0 < nkeys; c0 += 64) {
        const int64_t j = c0 + lane;
        const float s = allowed(j) ? score_of(key_of(j)) : -INFINITY;
        m = fmaxf(m, s);
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) m = fmaxf(m, __shfl_xor(m, o, 64));
    float acc[kAttnF32MaxHd / 64];
#pragma unroll
    for (int s = 0; s < kAttnF32MaxHd / 64; ++s) acc[s] = 0.0f;
    if (m != -INFINITY) {
        // Walk 2: the sum, in key order.
        float sum = 0.0f;
        for (int64_t c0 = 0; c0 < nkeys; c0 += 64) {
            const int64_t j = c0 + lane;
            const bool ok = allowed(j);
            const float e = ok ? expf(score_of(key_of(j)) - m) : 0.0f;
            const uint64_t okm = __ballot(ok);
            const int n = (int)(nkeys - c0 < 64 ? nkeys - c0 : 64);
            for (int jj = 0; jj < n; ++jj)
                if ((okm >> jj) & 1ull)
                    sum = sum + __uint_as_float(__builtin_amdgcn_readlane(__float_as_uint(e), jj));
        }
        // Walk 3: probabilities and the context, lane = dimension.
        for (int64_t c0 = 0; c0 < nkeys; c0 += 64) {
            const int64_t j = c0 + lane;
            const bool ok = allowed(j);
            const float p = ok ? expf(score_of(key_of(j)) - m) / sum : 0.0f;
            const uint64_t okm = __ballot(ok);
            const int n = (int)(nkeys - c0 < 64 ? nkeys - c0 : 64);
            for (int jj = 0; jj < n; ++jj) {
                if (!((okm >> jj) & 1ull)) continue;
                const float pj = __uint_as_float(__builtin_amdgcn_readlane(__float_as_uint(p), jj));
                const float* vr = vbase + key_of(c0 + jj) * kv_stride;
#pragma unroll
                for (int s = 0; s < kAttnF32MaxHd / 64; ++s) {
                    const int d = s * 64 + lane;
                    if (d < hd) acc[s] = acc[s] + pj * vr[d];
                }
            }
        }
    }
    float* orow = out + (b * T + qi) * out_stride + (int64_t)h * hd;
#pragma unroll
    for (int s = 0; s < kAttnF32MaxHd / 64; ++s) {
        const int d = s * 64 + lane;
        if (d < hd) orow[d] = acc[s];
    }
}

hipError_t launch_attention_f32(const float* q, const float* k, const float* v, float* out,
                                int64_t batch, int64_t T, int q_heads, int kv_heads, int hd,
                                int64_t q_stride, int64_t kv_stride, int64_t out_stride,
                                int64_t window, int64_t prefix, const int32_t* seg_lo,
                                const int32_t* seg_hi, const uint64_t* pad, hipStream_t st) {
    if (window >= T) window = 0;
    const dim3 grid((unsigned)T, (unsigned)((q_heads + 3) / 4), (unsigned)batch);
    hipLaunchKernelGGL(attention_f32_kernel, grid, dim3(256), 0, st, q, k, v, out, T, q_heads,
                       q_heads / kv_heads, hd, q_stride, kv_stride, out_stride, window,
                       1.0f / sqrtf((float)hd), prefix, seg_lo, seg_hi, pad);
    return hipGetLastError();
}

struct PlanF32 {
    int64_t T, q_w, kv_w;
    size_t o_hidden, o_normed, o_q, o_k, o_v, o_ctx, o_proj, o_gate, o_up, o_ids, total;
};

size_t up256(size_t v) { return (v + 255) & ~size_t(255); }

PlanF32 plan_f32(const ncm_decoder_shape_t& s, int64_t batch, int64_t seq) {
    PlanF32 p;
    p.T = batch * seq;
    p.q_w = (int64_t)s.q_heads * s.head_dim;
    p.kv_w = (int64_t)s.kv_heads * s.head_dim;
    size_t off = 0;
    auto carve = [&](size_t bytes) { const size_t o = off; off += up256(bytes); return o; };
    p.o_hidden = carve((size_t)p.T * s.hidden * 4);
    p.o_normed = carve((size_t)p.T * s.hidden * 4);
    p.o_q = carve((size_t)p.T * p.q_w * 4);
    p.o_k = carve((size_t)p.T * p.kv_w * 4);
    p.o_v = carve((size_t)p.T * p.kv_w * 4);
    p.o_ctx = carve((size_t)p.T * p.q_w * 4);
    p.o_proj = carve((size_t)p.T * s.hidden * 4);
    p.o_gate = carve((size_t)p.T * s.intermediate * 4);
    p.o_up = carve((size_t)p.T * s.intermediate * 4);
    p.o_ids = carve((size_t)p.T * 8);
    p.total = off;
    return p;
}

#define NCM_TRY(call)                                  \
    do {                                               \
        hipError_t e_ = (call);                        \
        if (e_ != hipSuccess) return e_;               \
    } while (0)

// Copies one stage [T, width] into trace layer `layer` (layer-major).
hipError_t trace_copy(float* dst, int layer, const float* src, int64_t T, int64_t width,
                      hipStream_t st) {
    if (!dst) return hipSuccess;
    const size_t bytes = (size_t)T * width * 4;
    return hipMemcpyAsync(dst + (int64_t)layer * T * width, src, bytes,
                          hipMemcpyDeviceToDevice, st);
}

}  // namespace

hipError_t launch_add_f32(float* y, const float* a, int64_t rows, int64_t n, int64_t a_rows,
                          hipStream_t st) {
    const int64_t total = rows * n;
    if (total == 0) return hipSuccess;
    hipLaunchKernelGGL(add_f32_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, st, y,
                       a, rows, n, a_rows);
    return hipGetLastError();
}

// y [rows, n] = x [rows, k] w^T (+ bias), f32.
hipError_t project_f32(const float* x, const float* w, const float* bias, float* y, int64_t rows,
                       int64_t k, int64_t n, hipStream_t st) {
    NCM_TRY(launch_linear_f32(x, w, y, rows, k, n, st));
    if (bias) NCM_TRY(launch_add_f32(y, bias, rows, n, 1, st));
    return hipSuccess;
}

hipError_t run_layers_f32(const LayerStackF32& a, hipStream_t st) {
    const ncm_decoder_shape_t& s = *a.shape;
    const int64_t T = a.batch * a.seq, H = s.hidden, I = s.intermediate;
    const int hd = s.head_dim;
    const int64_t q_w = (int64_t)s.q_heads * hd, kv_w = (int64_t)s.kv_heads * hd;
    const ncm_decoder_trace_t none{};
    const ncm_decoder_trace_t& tr = a.trace ? *a.trace : none;
    float *hidden = a.hidden, *normed = a.normed, *q = a.q, *k = a.k, *v = a.v, *ctx = a.ctx;
    float *proj = a.proj, *gate = a.gate, *up = a.up;
    for (int l = 0; l < s.layers; ++l) {
        const ncm_decoder_layer_f32_t& L = a.layers[l];
        NCM_TRY(launch_rms_norm_rows(hidden, L.input_norm, normed, T, H, s.rms_eps, NCM_OUT_F32,
                                     st));
        if (L.input_norm_bias) NCM_TRY(launch_add_f32(normed, L.input_norm_bias, T, H, 1, st));
        NCM_TRY(trace_copy(tr.input_norm, l, normed, T, H, st));
        const float* wq = L.qkv_weight;
        const float* wk = wq + q_w * H;
        const float* wv = wk + kv_w * H;
        const float* bq = L.qkv_bias;
        NCM_TRY(project_f32(normed, wq, bq, q, T, H, q_w, st));
        NCM_TRY(project_f32(normed, wk, bq ? bq + q_w : nullptr, k, T, H, kv_w, st));
        NCM_TRY(project_f32(normed, wv, bq ? bq + q_w + kv_w : nullptr, v, T, H, kv_w, st));
        if (L.q_norm) {  // QK-norm (f32 rms_norm of every head) before the rotation
            NCM_TRY(launch_rms_norm_rows(q, L.q_norm, q, T * s.q_heads, hd, s.rms_eps,
                                         NCM_OUT_F32, st));
            NCM_TRY(launch_rms_norm_rows(k, L.k_norm, k, T * s.kv_heads, hd, s.rms_eps,
                                         NCM_OUT_F32, st));
        }
        NCM_TRY(launch_rope_rotate_f32(q, T, q_w, s.q_heads, hd, a.seq, a.cosine, a.sine, st));
        NCM_TRY(launch_rope_rotate_f32(k, T, kv_w, s.kv_heads, hd, a.seq, a.cosine, a.sine, st));
        NCM_TRY(launch_attention_f32(q, k, v, ctx, a.batch, a.seq, s.q_heads, s.kv_heads, hd, q_w,
                                     kv_w, q_w, a.seg_lo ? 0 : s.window, a.prefix, a.seg_lo,
                                     a.seg_hi, a.pad, st));
        NCM_TRY(trace_copy(tr.attention_context, l, ctx, T, q_w, st));
        NCM_TRY(project_f32(ctx, L.o_weight, L.o_bias, proj, T, q_w, H, st));
        NCM_TRY(trace_copy(tr.attention_output, l, proj, T, H, st));
        NCM_TRY(launch_add_f32(hidden, proj, T, H, T, st));
        NCM_TRY(trace_copy(tr.attention_residual, l, hidden, T, H, st));
        NCM_TRY(launch_rms_norm_rows(hidden, L.post_attention_norm, normed, T, H, s.rms_eps,
                                     NCM_OUT_F32, st));
        if (L.post_attention_norm_bias)
            NCM_TRY(launch_add_f32(normed, L.post_attention_norm_bias, T, H, 1, st));
        NCM_TRY(trace_copy(tr.post_attention_norm, l, normed, T, H, st));
        NCM_TRY(project_f32(normed, L.gate_weight, L.gate_bias, gate, T, H, I, st));
        NCM_TRY(trace_copy(tr.gate_projection, l, gate, T, I, st));
        NCM_TRY(project_f32(normed, L.up_weight, L.up_bias, up, T, H, I, st));
        NCM_TRY(trace_copy(tr.up_projection, l, up, T, I, st));
        NCM_TRY(launch_silu_mul(gate, up, gate, T * I, NCM_OUT_F32, st));
        NCM_TRY(trace_copy(tr.gate_up_product, l, gate, T, I, st));
        NCM_TRY(project_f32(gate, L.down_weight, L.down_bias, proj, T, I, H, st));
        NCM_TRY(trace_copy(tr.mlp_output, l, proj, T, H, st));
        NCM_TRY(launch_add_f32(hidden, proj, T, H, T, st));
        NCM_TRY(trace_copy(tr.block_output, l, hidden, T, H, st));
    }
    return hipSuccess;
}

size_t decoder_f32_workspace_bytes(const ncm_decoder_shape_t& s, int64_t batch, int64_t seq) {
    return plan_f32(s, batch, seq).total;
}

hipError_t decoder_forward_f32(const ncm_decoder_shape_t& s, const ncm_decoder_layer_f32_t* layers,
                               const float* embed, const float* final_norm, const float* lm_head,
                               const float* cosine, const float* sine, const int64_t* host_ids,
                               int64_t batch, int64_t seq, float* logits,
                               const ncm_decoder_trace_t* trace, void* ws, hipStream_t st) {
    const PlanF32 p = plan_f32(s, batch, seq);
    char* w = (char*)ws;
    float* hidden = (float*)(w + p.o_hidden);
    float* normed = (float*)(w + p.o_normed);
    float* q = (float*)(w + p.o_q);
    float* k = (float*)(w + p.o_k);
    float* v = (float*)(w + p.o_v);
    float* ctx = (float*)(w + p.o_ctx);
    float* proj = (float*)(w + p.o_proj);
    float* gate = (float*)(w + p.o_gate);
    float* up = (float*)(w + p.o_up);
    int64_t* ids = (int64_t*)(w + p.o_ids);
    const int64_t T = p.T, H = s.hidden;
    const ncm_decoder_trace_t none{};
    const ncm_decoder_trace_t& tr = trace ? *trace : none;

    NCM_TRY(hipMemcpyAsync(ids, host_ids, (size_t)T * 8, hipMemcpyHostToDevice, st));
    {
        const dim3 grid((unsigned)((H + 255) / 256 < 64 ? (H + 255) / 256 : 64), (unsigned)T);
        hipLaunchKernelGGL(embed_rows_f32_kernel, grid, dim3(256), 0, st, ids, embed, hidden, H);
        NCM_TRY(hipGetLastError());
    }
    NCM_TRY(trace_copy(tr.block_input, 0, hidden, T, H, st));
    LayerStackF32 a{};
    a.shape = &s;
    a.layers = layers;
    a.batch = batch;
    a.seq = seq;
    a.cosine = cosine;
    a.sine = sine;
    a.hidden = hidden; a.normed = normed; a.q = q; a.k = k; a.v = v; a.ctx = ctx;
    a.proj = proj; a.gate = gate; a.up = up;
    a.trace = trace;
    NCM_TRY(run_layers_f32(a, st));
    NCM_TRY(launch_rms_norm_rows(hidden, final_norm, normed, T, H, s.rms_eps, NCM_OUT_F32, st));
    NCM_TRY(launch_linear_f32(normed, lm_head ? lm_head : embed, logits, T, H, s.vocab, st));
    return hipSuccess;
}

}  // namespace ncm
