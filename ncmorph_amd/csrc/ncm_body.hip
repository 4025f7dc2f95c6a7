// The NCM level-parallel body (forward_with_trace, src/ncm_model.zig:89-250)
// in the bf16 mode of the source decoder, on one GPU:
//   rows     = [prefix_token_embedding[ids] | target_inputs], level 0's rows
//              replaced by l0_queries when query_level0        (fp32)
//   rows    += Conv1d(rows) per level, when convolutions are given
//              (apply_post_upsample_conv, :296-326; fp32 on the fp32 MFMA)
//   h        = round(bf16(rows) W_in^T + bias)     (matmul_bf16_bias, flushed operands)
//   h[level] = round(h + level_embedding[level])   (use_level_encoding)
//   h        = the decoder's bf16 layer stack (run_layers) with the block-
//              diagonal (reference) or block-causal level mask, or the causal
//              one (source_causal), RoPE at positions restarting per level
//   out      = rms_norm_bf16(h, final_norm) (+ bias, rounded)
// The reference runs this body in f32 (kernels.matmul, f32 attention); the
// bf16 rules are those decoder.zig applies with bf16_compute.
#include <hip/hip_runtime.h>

#include <vector>

#include "common.h"
#include "decoder.h"
#include "linear.h"
#include "ncm_body.h"

namespace ncm {

// out[r] (fp32, width vq): the prefix table row of ids[r] (r < P), a
// learned level-0 query (P <= r < P + l0_rows), else target row r - P.
// Tables of bf16 bits (bf16 body) or floats (f32 body).
__device__ __forceinline__ float table_value(const uint16_t* t, int64_t i) {
    return __uint_as_float((uint32_t)t[i] << 16);
}
__device__ __forceinline__ float table_value(const float* t, int64_t i) { return t[i]; }

template <class TT>
__global__ __launch_bounds__(256) void ncm_input_rows_kernel(
    const int64_t* __restrict__ ids, const TT* __restrict__ table, const TT* __restrict__ l0,
    const float* __restrict__ target, float* __restrict__ out, int64_t P, int64_t l0_rows,
    int64_t S, int64_t vq) {
    for (int64_t r = blockIdx.y; r < S; r += gridDim.y) {
        float* dst = out + r * vq;
        for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < vq;
             i += (int64_t)gridDim.x * 256) {
            float v;
            if (r < P)
                v = table_value(table, ids[r] * vq + i);
            else if (r - P < l0_rows)
                v = table_value(l0, (r - P) * vq + i);
            else
                v = target[(r - P) * vq + i];
            dst[i] = v;
        }
    }
}

// col[p, 3 i + k] = x[p + k - 1, i] (zero outside the level's rows): the
// 3-tap Conv1d as a product with the reference's [out][in][3] weights.
__global__ __launch_bounds__(256) void conv_im2col_kernel(const float* __restrict__ x,
                                                          float* __restrict__ col, int64_t rows,
                                                          int64_t width) {
    const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (idx >= rows * width * 3) return;
    const int64_t p = idx / (3 * width);
    const int64_t j = idx % (3 * width);
    const int64_t i = j / 3, k = j % 3;
    const int64_t src = p + k - 1;
    col[idx] = (src >= 0 && src < rows) ? x[src * width + i] : 0.0f;
}

// x = x + (y + bias): the residual of the post-upsample convolution.
__global__ __launch_bounds__(256) void conv_finish_kernel(float* __restrict__ x,
                                                          const float* __restrict__ y,
                                                          const float* __restrict__ bias,
                                                          int64_t rows, int64_t width) {
    const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (idx >= rows * width) return;
    x[idx] = x[idx] + (y[idx] + bias[idx % width]);
}

struct LevelTableArgs {
    int64_t begin[kMaxNcmLevels + 1];  // row where each level starts; begin[n] = S
    int32_t n;
};

// h[r] = round_bf16(h[r] + level_embedding[level of r]) for target rows.
__global__ __launch_bounds__(256) void level_embed_kernel(float* __restrict__ h,
                                                          const uint16_t* __restrict__ emb,
                                                          LevelTableArgs lt, int64_t H) {
    for (int64_t r = lt.begin[0] + blockIdx.y; r < lt.begin[lt.n]; r += gridDim.y) {
        int l = 0;
        while (l + 1 < lt.n && r >= lt.begin[l + 1]) ++l;
        float* row = h + r * H;
        const uint16_t* e = emb + (int64_t)l * H;
        for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < H;
             i += (int64_t)gridDim.x * 256)
            row[i] = __uint_as_float(
                bf16_bits_rne(row[i] + __uint_as_float((uint32_t)e[i] << 16)) << 16);
    }
}

// h[r] = h[r] + level_embedding[level of r] for target rows, f32 (no rounding).
__global__ __launch_bounds__(256) void level_embed_f32_kernel(float* __restrict__ h,
                                                              const float* __restrict__ emb,
                                                              LevelTableArgs lt, int64_t H) {
    for (int64_t r = lt.begin[0] + blockIdx.y; r < lt.begin[lt.n]; r += gridDim.y) {
        int l = 0;
        while (l + 1 < lt.n && r >= lt.begin[l + 1]) ++l;
        float* row = h + r * H;
        const float* e = emb + (int64_t)l * H;
        for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < H;
             i += (int64_t)gridDim.x * 256)
            row[i] = row[i] + e[i];
    }
}

namespace {

constexpr size_t kAlign = 256;
size_t up(size_t n) { return (n + kAlign - 1) / kAlign * kAlign; }

struct NcmPlan {
    int64_t S, T, max_level;
    size_t o_rows, o_rows16, o_col, o_convy, o_hidden, o_normed, o_qkv, o_ctx, o_act, o_ids,
        o_seg_lo, o_seg_hi, o_pad, o_vt, total;
};

NcmPlan ncm_plan(const ncm_ncm_shape_t& s, bool convs) {
    NcmPlan p{};
    p.T = 0;
    p.max_level = 0;
    for (int l = 0; l < s.n_levels; ++l) {
        p.T += s.level_lengths[l];
        if (s.level_lengths[l] > p.max_level) p.max_level = s.level_lengths[l];
    }
    p.S = s.prefix_length + p.T;
    const int64_t qkv_w = (int64_t)(s.q_heads + 2 * s.kv_heads) * s.head_dim;
    const int64_t q_w = (int64_t)s.q_heads * s.head_dim;
    size_t off = 0;
    auto carve = [&](size_t bytes) { const size_t o = off; off += up(bytes); return o; };
    p.o_rows = carve((size_t)p.S * s.vq_width * 4);
    p.o_rows16 = carve((size_t)p.S * s.vq_width * 2);
    p.o_col = carve(convs ? (size_t)p.max_level * 3 * s.vq_width * 4 : 0);
    p.o_convy = carve(convs ? (size_t)p.max_level * s.vq_width * 4 : 0);
    p.o_hidden = carve((size_t)p.S * s.hidden * 4);
    p.o_normed = carve((size_t)p.S * s.hidden * 2);
    p.o_qkv = carve((size_t)p.S * qkv_w * 2);
    p.o_ctx = carve((size_t)p.S * q_w * 2);
    p.o_act = carve((size_t)p.S * s.intermediate * 2);
    p.o_ids = carve((size_t)(s.prefix_length > 0 ? s.prefix_length : 1) * 8);
    p.o_seg_lo = carve((size_t)p.S * 4);
    p.o_seg_hi = carve((size_t)p.S * 4);
    p.o_pad = carve((size_t)((s.prefix_length + 63) / 64 + 1) * 8);
    p.o_vt = carve(attention_workspace_bytes(1, p.S, s.kv_heads, s.head_dim));
    p.total = off;
    return p;
}

#define NCM_TRY(call)                                  \
    do {                                               \
        hipError_t e_ = (call);                        \
        if (e_ != hipSuccess) return e_;               \
    } while (0)

}  // namespace

namespace {

// Host-built inputs: the level table, the level mask's per-position key
// range (block-diagonal: the own level; block-causal: every level up to the
// own one; prefix rows: none) and the prefix pad bits.
struct HostInputs {
    std::vector<int32_t> lo, hi;
    std::vector<uint64_t> bits;
    LevelTableArgs lt;
};

HostInputs host_inputs(const ncm_ncm_shape_t& s, const uint8_t* host_pad, int64_t pad_len) {
    HostInputs h;
    const int64_t P = s.prefix_length;
    int64_t S = P;
    for (int l = 0; l < s.n_levels; ++l) S += s.level_lengths[l];
    h.lo.assign((size_t)S, 0);
    h.hi.assign((size_t)S, 0);
    h.lt = LevelTableArgs{};
    h.lt.n = s.n_levels;
    int64_t off = P;
    for (int l = 0; l < s.n_levels; ++l) {
        h.lt.begin[l] = off;
        for (int64_t t = off; t < off + s.level_lengths[l]; ++t) {
            h.lo[(size_t)t] = (int32_t)(s.mask_mode == NCM_MASK_BLOCK_CAUSAL ? P : off);
            h.hi[(size_t)t] = (int32_t)(off + s.level_lengths[l]);
        }
        off += s.level_lengths[l];
    }
    h.lt.begin[s.n_levels] = off;
    h.bits.assign((size_t)((P + 63) / 64 + 1), 0ull);
    for (int64_t t = 0; t < pad_len; ++t)
        if (host_pad[t]) h.bits[(size_t)(t / 64)] |= 1ull << (t % 64);
    return h;
}

// Prefix ids, key ranges and pad bits to the device. Pageable copies: the
// host vectors may go once the calls return.
hipError_t upload_inputs(const ncm_ncm_shape_t& s, const HostInputs& h, const int64_t* host_ids,
                         int64_t* ids, int32_t* seg_lo, int32_t* seg_hi, uint64_t* pad,
                         hipStream_t st) {
    const int64_t P = s.prefix_length;
    if (P > 0) NCM_TRY(hipMemcpyAsync(ids, host_ids, (size_t)P * 8, hipMemcpyHostToDevice, st));
    if (s.mask_mode != NCM_MASK_CAUSAL) {
        NCM_TRY(hipMemcpyAsync(seg_lo, h.lo.data(), h.lo.size() * 4, hipMemcpyHostToDevice, st));
        NCM_TRY(hipMemcpyAsync(seg_hi, h.hi.data(), h.hi.size() * 4, hipMemcpyHostToDevice, st));
        NCM_TRY(hipMemcpyAsync(pad, h.bits.data(), h.bits.size() * 8, hipMemcpyHostToDevice, st));
    }
    return hipSuccess;
}

template <class TT>
hipError_t input_rows(const ncm_ncm_shape_t& s, const int64_t* ids, const TT* table,
                      const TT* l0, const float* target, float* rows, hipStream_t st) {
    int64_t S = s.prefix_length;
    for (int l = 0; l < s.n_levels; ++l) S += s.level_lengths[l];
    const int64_t vq = s.vq_width;
    const unsigned gx = (unsigned)((vq + 255) / 256 < 16 ? (vq + 255) / 256 : 16);
    const int64_t l0_rows = s.query_level0 ? s.level_lengths[0] : 0;
    const unsigned gy = (unsigned)(S < 65535 ? S : 65535);
    hipLaunchKernelGGL(ncm_input_rows_kernel<TT>, dim3(gx, gy), dim3(256), 0, st, ids, table, l0,
                       target, rows, s.prefix_length, l0_rows, S, vq);
    return hipGetLastError();
}

// rows[level] += Conv1d(rows[level]) + bias for every level (fp32 MFMA).
hipError_t apply_convs(const ncm_ncm_shape_t& s, const LevelTableArgs& lt, float* rows,
                       float* col, float* cy, const float* const* cw, const float* const* cb,
                       hipStream_t st) {
    const int64_t vq = s.vq_width;
    for (int l = 0; l < s.n_levels; ++l) {
        const int64_t n = s.level_lengths[l];
        if (n == 0) continue;
        float* x = rows + lt.begin[l] * vq;
        hipLaunchKernelGGL(conv_im2col_kernel, dim3((unsigned)((n * vq * 3 + 255) / 256)),
                           dim3(256), 0, st, x, col, n, vq);
        NCM_TRY(hipGetLastError());
        NCM_TRY(launch_linear_f32(col, cw[l], cy, n, 3 * vq, vq, st));
        hipLaunchKernelGGL(conv_finish_kernel, dim3((unsigned)((n * vq + 255) / 256)), dim3(256),
                           0, st, x, cy, cb[l], n, vq);
        NCM_TRY(hipGetLastError());
    }
    return hipSuccess;
}

}  // namespace

size_t ncm_workspace_bytes(const ncm_ncm_shape_t& s, bool convs) {
    return ncm_plan(s, convs).total;
}

hipError_t ncm_forward(const ncm_ncm_shape_t& s, const ncm_decoder_layer_t* layers,
                       const ncm_ncm_weights_t& w, const int64_t* host_ids,
                       const uint8_t* host_pad, int64_t pad_len, const float* target,
                       const float* cosine, const float* sine, float* output,
                       float* hidden_states, void* ws, hipStream_t st) {
    const bool convs = w.conv_weight != nullptr;
    const NcmPlan p = ncm_plan(s, convs);
    char* base = (char*)ws;
    float* rows = (float*)(base + p.o_rows);
    uint16_t* rows16 = (uint16_t*)(base + p.o_rows16);
    int64_t* ids = (int64_t*)(base + p.o_ids);
    int32_t* seg_lo = (int32_t*)(base + p.o_seg_lo);
    int32_t* seg_hi = (int32_t*)(base + p.o_seg_hi);
    uint64_t* pad = (uint64_t*)(base + p.o_pad);
    const int64_t P = s.prefix_length, S = p.S, vq = s.vq_width, H = s.hidden;

    const HostInputs hi_ = host_inputs(s, host_pad, pad_len);
    const LevelTableArgs& lt = hi_.lt;
    const bool levels_mask = s.mask_mode != NCM_MASK_CAUSAL;
    NCM_TRY(upload_inputs(s, hi_, host_ids, ids, seg_lo, seg_hi, pad, st));

    // Input rows (fp32), then the per-level convolutions in place.
    NCM_TRY(input_rows<uint16_t>(s, ids, w.prefix_token_embedding, w.l0_queries, target, rows,
                                 st));
    if (convs)
        NCM_TRY(apply_convs(s, lt, rows, (float*)(base + p.o_col), (float*)(base + p.o_convy),
                            w.conv_weight, w.conv_bias, st));
    // bf16 operands as matmul_bf16 forms them (RNE, subnormals flushed).
    NCM_TRY(launch_bf16_from_f32(rows, rows16, S * vq, 1, st));

    LayerStack a{};
    ncm_decoder_shape_t ds{};
    ds.hidden = H;
    ds.intermediate = s.intermediate;
    ds.vocab = 1;
    ds.q_heads = s.q_heads;
    ds.kv_heads = s.kv_heads;
    ds.head_dim = s.head_dim;
    ds.layers = s.layers;
    ds.window = s.mask_mode == NCM_MASK_CAUSAL ? s.window : 0;
    ds.rms_eps = s.rms_eps;
    a.shape = &ds;
    a.layers = layers;
    a.batch = 1;
    a.seq = S;
    a.cosine = cosine;
    a.sine = sine;
    a.prefix = P;
    a.seg_lo = levels_mask ? seg_lo : nullptr;
    a.seg_hi = levels_mask ? seg_hi : nullptr;
    a.pad = levels_mask && pad_len > 0 ? pad : nullptr;
    a.hidden = (float*)(base + p.o_hidden);
    a.normed = (uint16_t*)(base + p.o_normed);
    a.qkv = (uint16_t*)(base + p.o_qkv);
    a.ctx = (uint16_t*)(base + p.o_ctx);
    a.act = (uint16_t*)(base + p.o_act);
    a.vt = (uint16_t*)(base + p.o_vt);

    NCM_TRY(launch_linear(rows16, w.input_projection, w.input_projection_bias, a.hidden, S, vq, H,
                          NCM_OUT_BF16_F32, -1, st));
    if (s.use_level_encoding && p.T > 0) {
        const unsigned gx = (unsigned)((H + 255) / 256 < 16 ? (H + 255) / 256 : 16);
        const unsigned gy = (unsigned)(p.T < 65535 ? p.T : 65535);
        hipLaunchKernelGGL(level_embed_kernel, dim3(gx, gy), dim3(256), 0, st, a.hidden,
                           w.level_embedding, lt, H);
        NCM_TRY(hipGetLastError());
    }
    // hidden_states [layers + 1, S, H] (src/ncm_model.zig:169-171, :243-249):
    // the input stage, each layer's output (the last one's place then takes
    // the final-normalized output).
    ncm_decoder_trace_t tr{};
    if (hidden_states) {
        NCM_TRY(hipMemcpyAsync(hidden_states, a.hidden, (size_t)S * H * 4,
                               hipMemcpyDeviceToDevice, st));
        tr.block_output = hidden_states + S * H;
        a.trace = &tr;
    }
    NCM_TRY(run_layers(a, st));
    NCM_TRY(launch_rms_norm_rows(a.hidden, w.final_norm, output, S, H, s.rms_eps,
                                 NCM_OUT_BF16_F32, st));
    if (w.final_norm_bias) NCM_TRY(launch_bias_round(output, w.final_norm_bias, S, H, false, st));
    if (hidden_states)
        NCM_TRY(hipMemcpyAsync(hidden_states + (int64_t)s.layers * S * H, output,
                               (size_t)S * H * 4, hipMemcpyDeviceToDevice, st));
    return hipSuccess;
}


namespace {

struct NcmPlanF32 {
    int64_t S, T, max_level;
    size_t o_rows, o_col, o_convy, o_hidden, o_normed, o_q, o_k, o_v, o_ctx, o_proj, o_gate,
        o_up, o_ids, o_seg_lo, o_seg_hi, o_pad, total;
};

NcmPlanF32 ncm_plan_f32(const ncm_ncm_shape_t& s, bool convs) {
    NcmPlanF32 p{};
    for (int l = 0; l < s.n_levels; ++l) {
        p.T += s.level_lengths[l];
        if (s.level_lengths[l] > p.max_level) p.max_level = s.level_lengths[l];
    }
    p.S = s.prefix_length + p.T;
    const int64_t q_w = (int64_t)s.q_heads * s.head_dim;
    const int64_t kv_w = (int64_t)s.kv_heads * s.head_dim;
    size_t off = 0;
    auto carve = [&](size_t bytes) { const size_t o = off; off += up(bytes); return o; };
    const size_t S = (size_t)p.S;
    p.o_rows = carve(S * s.vq_width * 4);
    p.o_col = carve(convs ? (size_t)p.max_level * 3 * s.vq_width * 4 : 0);
    p.o_convy = carve(convs ? (size_t)p.max_level * s.vq_width * 4 : 0);
    p.o_hidden = carve(S * s.hidden * 4);
    p.o_normed = carve(S * s.hidden * 4);
    p.o_q = carve(S * q_w * 4);
    p.o_k = carve(S * kv_w * 4);
    p.o_v = carve(S * kv_w * 4);
    p.o_ctx = carve(S * q_w * 4);
    p.o_proj = carve(S * s.hidden * 4);
    p.o_gate = carve(S * s.intermediate * 4);
    p.o_up = carve(S * s.intermediate * 4);
    p.o_ids = carve((size_t)(s.prefix_length > 0 ? s.prefix_length : 1) * 8);
    p.o_seg_lo = carve(S * 4);
    p.o_seg_hi = carve(S * 4);
    p.o_pad = carve((size_t)((s.prefix_length + 63) / 64 + 1) * 8);
    p.total = off;
    return p;
}

}  // namespace

size_t ncm_f32_workspace_bytes(const ncm_ncm_shape_t& s, bool convs) {
    return ncm_plan_f32(s, convs).total;
}

// The body in the reference's arithmetic (forward_with_trace,
// src/ncm_model.zig:89-250, f32 throughout):
//   rows  = [prefix_token_embedding[ids] | target_inputs] (level 0 from
//           l0_queries when query_level0), += Conv1d per level
//   h     = rows W_in^T + bias                     (kernels.matmul, :278-294)
//   h[level] += level_embedding[level]
//   h     = the f32 layer stack (run_layers_f32) with the level mask
//   out   = rms_norm(h, final_norm) + final_norm_bias (ncm_norm.zig:22-49)
hipError_t ncm_forward_f32(const ncm_ncm_shape_t& s, const ncm_decoder_layer_f32_t* layers,
                           const ncm_ncm_weights_f32_t& w, const int64_t* host_ids,
                           const uint8_t* host_pad, int64_t pad_len, const float* target,
                           const float* cosine, const float* sine, float* output,
                           float* hidden_states, void* ws, hipStream_t st) {
    const bool convs = w.conv_weight != nullptr;
    const NcmPlanF32 p = ncm_plan_f32(s, convs);
    char* base = (char*)ws;
    float* rows = (float*)(base + p.o_rows);
    int64_t* ids = (int64_t*)(base + p.o_ids);
    int32_t* seg_lo = (int32_t*)(base + p.o_seg_lo);
    int32_t* seg_hi = (int32_t*)(base + p.o_seg_hi);
    uint64_t* pad = (uint64_t*)(base + p.o_pad);
    const int64_t S = p.S, vq = s.vq_width, H = s.hidden;

    const HostInputs hin = host_inputs(s, host_pad, pad_len);
    const bool levels_mask = s.mask_mode != NCM_MASK_CAUSAL;
    NCM_TRY(upload_inputs(s, hin, host_ids, ids, seg_lo, seg_hi, pad, st));
    NCM_TRY(input_rows<float>(s, ids, w.prefix_token_embedding, w.l0_queries, target, rows, st));
    if (convs)
        NCM_TRY(apply_convs(s, hin.lt, rows, (float*)(base + p.o_col), (float*)(base + p.o_convy),
                            w.conv_weight, w.conv_bias, st));

    LayerStackF32 a{};
    ncm_decoder_shape_t ds{};
    ds.hidden = H;
    ds.intermediate = s.intermediate;
    ds.vocab = 1;
    ds.q_heads = s.q_heads;
    ds.kv_heads = s.kv_heads;
    ds.head_dim = s.head_dim;
    ds.layers = s.layers;
    ds.window = s.mask_mode == NCM_MASK_CAUSAL ? s.window : 0;
    ds.rms_eps = s.rms_eps;
    a.shape = &ds;
    a.layers = layers;
    a.batch = 1;
    a.seq = S;
    a.cosine = cosine;
    a.sine = sine;
    a.prefix = s.prefix_length;
    a.seg_lo = levels_mask ? seg_lo : nullptr;
    a.seg_hi = levels_mask ? seg_hi : nullptr;
    a.pad = levels_mask && pad_len > 0 ? pad : nullptr;
    a.hidden = (float*)(base + p.o_hidden);
    a.normed = (float*)(base + p.o_normed);
    a.q = (float*)(base + p.o_q);
    a.k = (float*)(base + p.o_k);
    a.v = (float*)(base + p.o_v);
    a.ctx = (float*)(base + p.o_ctx);
    a.proj = (float*)(base + p.o_proj);
    a.gate = (float*)(base + p.o_gate);
    a.up = (float*)(base + p.o_up);
    a.trace = nullptr;

    NCM_TRY(project_f32(rows, w.input_projection, w.input_projection_bias, a.hidden, S, vq, H, st));
    if (s.use_level_encoding && p.T > 0) {
        const unsigned gx = (unsigned)((H + 255) / 256 < 16 ? (H + 255) / 256 : 16);
        const unsigned gy = (unsigned)(p.T < 65535 ? p.T : 65535);
        hipLaunchKernelGGL(level_embed_f32_kernel, dim3(gx, gy), dim3(256), 0, st, a.hidden,
                           w.level_embedding, hin.lt, H);
        NCM_TRY(hipGetLastError());
    }
    // hidden_states as in ncm_forward.
    ncm_decoder_trace_t tr{};
    if (hidden_states) {
        NCM_TRY(hipMemcpyAsync(hidden_states, a.hidden, (size_t)S * H * 4,
                               hipMemcpyDeviceToDevice, st));
        tr.block_output = hidden_states + S * H;
        a.trace = &tr;
    }
    NCM_TRY(run_layers_f32(a, st));
    NCM_TRY(launch_rms_norm_rows(a.hidden, w.final_norm, output, S, H, s.rms_eps, NCM_OUT_F32,
                                 st));
    if (w.final_norm_bias) NCM_TRY(launch_add_f32(output, w.final_norm_bias, S, H, 1, st));
    if (hidden_states)
        NCM_TRY(hipMemcpyAsync(hidden_states + (int64_t)s.layers * S * H, output,
                               (size_t)S * H * 4, hipMemcpyDeviceToDevice, st));
    return hipSuccess;
}

}  // namespace ncm
