// Causal bf16 attention for the decoder's prefill (packages/kernels/root.zig:
// 536-578, softmax :272-284, mask :380-399), after the q/k/v projections and
// the rotation. Per query and head, in the reference's bf16 mode:
//   s_k = round(round(q . k_k) * 1/sqrt(head_dim))   (k allowed by the mask)
//   p_k = round(exp(s_k - max s) / sum exp(s - max s))
//   context = round(sum_k p_k v_k)
// Every value entering a product is bf16, so q . k and p v are sums of exact
// fp32 products; the MFMA sums them in its own order instead of the
// reference's key order, and the softmax sum is kept online. Results agree
// with the reference within a few bf16 steps, not bit for bit.
//
// Two passes over the key blocks of one (sequence, head, 128 queries)
// workgroup: pass 1 finds max s and the softmax sum; pass 2 recomputes the
// scores, forms the bf16 probabilities and accumulates P V. Keys are
// processed in blocks of 64: K rows staged in LDS (row-padded), V staged
// transposed (one LDS row per head dimension) so that each lane's eight
// P-operand keys are two 8-byte LDS reads.
//
// Scores are computed transposed, S^T = K Q^T, with v_mfma_f32_32x32x16_bf16:
// lane l then holds query l % 32 and keys 8 (i / 4) + 4 (l / 32) + i % 4 of a
// 32-key tile in element i. Elements 8j .. 8j+7 of that fragment are exactly
// the A operand of P V for the keys 16j + {4h .. 4h+3, 8+4h .. 8+4h+3}
// (h = l / 32); the V operand is read for the same keys, so the sum runs
// over the right pairs without moving P between lanes.
#include "common.h"
#include "linear.h"

namespace ncm {

namespace {

constexpr int kBq = 128;  // queries per workgroup (32 per wave)
constexpr int kBk = 64;   // keys per block

__device__ __forceinline__ float round_bf16_f(float v) {
    return __uint_as_float(bf16_bits_rne(v) << 16);
}

template <int HD>
struct AttnLds {
    static constexpr int KROW = HD * 2 + 16;   // bytes per staged K row
    static constexpr int VROW = kBk * 2 + 8;   // bytes per staged V^T row (one dim)
    static constexpr int K_BYTES = kBk * KROW;
    static constexpr int V_BYTES = HD * VROW;
};

// K block [kBk keys][HD] -> LDS rows; keys at or past `valid` are zero.
template <int HD>
__device__ __forceinline__ void stage_k(char* kl, const uint16_t* kbase, int64_t kv_stride,
                                        int64_t key0, int64_t valid) {
    constexpr int CPR = HD / 8;  // 16-byte chunks per row
#pragma unroll
    for (int j = 0; j < kBk * CPR / 256; ++j) {
        const int chunk = threadIdx.x + 256 * j;
        const int row = chunk / CPR, cc = chunk % CPR;
        u32x4_t val = {0u, 0u, 0u, 0u};
        if (key0 + row < valid)
            val = *(const u32x4_t*)(kbase + (key0 + row) * kv_stride + 8 * cc);
        *(u32x4_t*)(kl + row * AttnLds<HD>::KROW + 16 * cc) = val;
    }
}

// V block [kBk keys][HD] -> LDS V^T [HD][kBk] (keys at or past `valid` zero).
// Task (key pair kp, dim chunk dc): two 16-byte global loads, eight 4-byte
// LDS stores; consecutive threads take consecutive key pairs, so a wave's
// stores to one V^T row are contiguous.
template <int HD>
__device__ __forceinline__ void stage_v(char* vl, const uint16_t* vbase, int64_t kv_stride,
                                        int64_t key0, int64_t valid) {
    constexpr int TASKS = (kBk / 2) * (HD / 8);
#pragma unroll
    for (int j = 0; j < TASKS / 256; ++j) {
        const int task = threadIdx.x + 256 * j;
        const int kp = task % (kBk / 2), dc = task / (kBk / 2);
        const int64_t k0 = key0 + 2 * kp;
        u32x4_t a = {0u, 0u, 0u, 0u}, b = {0u, 0u, 0u, 0u};
        if (k0 < valid) a = *(const u32x4_t*)(vbase + k0 * kv_stride + 8 * dc);
        if (k0 + 1 < valid) b = *(const u32x4_t*)(vbase + (k0 + 1) * kv_stride + 8 * dc);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const uint32_t lo = (a[e] & 0xFFFFu) | (b[e] << 16);
            const uint32_t hi = (a[e] >> 16) | (b[e] & 0xFFFF0000u);
            *(uint32_t*)(vl + (8 * dc + 2 * e) * AttnLds<HD>::VROW + 4 * kp) = lo;
            *(uint32_t*)(vl + (8 * dc + 2 * e + 1) * AttnLds<HD>::VROW + 4 * kp) = hi;
        }
    }
}

// S^T tile pair for one wave: keys key0 + [0, 64) x this wave's 32 queries.
template <int HD>
__device__ __forceinline__ void scores_t(const char* kl, const u32x4_t (&qf)[HD / 16],
                                         f32x16_t (&acc)[2], int lane) {
    const int c = lane & 31, hl = lane >> 5;
#pragma unroll
    for (int t = 0; t < 2; ++t) {
        f32x16_t a = {};
#pragma unroll
        for (int s = 0; s < HD / 16; ++s) {
            const u32x4_t kf =
                *(const u32x4_t*)(kl + (32 * t + c) * AttnLds<HD>::KROW + (16 * s + 8 * hl) * 2);
            a = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, kf),
                                                        __builtin_bit_cast(bf16x8_t, qf[s]), a,
                                                        0, 0, 0);
        }
        acc[t] = a;
    }
}

}  // namespace

template <int HD, int OUT_MODE>
__global__ __launch_bounds__(256) void attention_bf16_kernel(
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ k,
    const uint16_t* __restrict__ v, void* __restrict__ out, int64_t T, int group,
    int64_t q_stride, int64_t kv_stride, int64_t out_stride, int64_t window, float scale) {
    using L = AttnLds<HD>;
    __shared__ __attribute__((aligned(16))) char kl[L::K_BYTES];
    __shared__ __attribute__((aligned(16))) char vl[L::V_BYTES];

    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int c = lane & 31, hl = lane >> 5;
    const int64_t b = blockIdx.z;
    const int h = blockIdx.y, kvh = h / group;
    const int64_t q0 = (int64_t)blockIdx.x * kBq;
    const int64_t qw0 = q0 + 32 * wave;
    const int64_t qq = qw0 + c;  // the query of this lane's score column
    const uint16_t* kbase = k + b * T * kv_stride + (int64_t)kvh * HD;
    const uint16_t* vbase = v + b * T * kv_stride + (int64_t)kvh * HD;

    // Q as the B operand of K Q^T: query qq, dims 16 s + 8 hl .. + 7.
    u32x4_t qf[HD / 16];
    {
        const uint16_t* qrow = q + (b * T + qq) * q_stride + (int64_t)h * HD + 8 * hl;
#pragma unroll
        for (int s = 0; s < HD / 16; ++s)
            qf[s] = qq < T ? *(const u32x4_t*)(qrow + 16 * s) : u32x4_t{0u, 0u, 0u, 0u};
    }

    // Key blocks of the workgroup: keys <= its last query; with a window,
    // keys > (first query - window).
    const int64_t q_last = (q0 + kBq < T ? q0 + kBq : T) - 1;
    int64_t k_lo = window > 0 ? q0 - window + 1 : 0;
    if (k_lo < 0) k_lo = 0;
    const int64_t kb_begin = k_lo / kBk, kb_end = q_last / kBk + 1;
    // This wave's queries (up to T) and the keys they can see.
    const int64_t wq_last = (qw0 + 31 < T ? qw0 + 31 : T - 1);
    int64_t wk_lo = window > 0 ? qw0 - window + 1 : 0;
    if (wk_lo < 0) wk_lo = 0;
    const bool wave_live = qw0 < T;

    auto allowed = [&](int64_t key) {
        return key <= qq && key < T && (window <= 0 || key + window > qq);
    };
    auto score = [&](float acc) { return round_bf16_f(round_bf16_f(acc) * scale); };

    // ---- pass 1: running max and softmax sum per query.
    float m = -INFINITY, lsum = 0.0f;
    for (int64_t kb = kb_begin; kb < kb_end; ++kb) {
        const int64_t key0 = kb * kBk;
        stage_k<HD>(kl, kbase, kv_stride, key0, T);
        __syncthreads();
        if (wave_live && key0 <= wq_last && key0 + kBk > wk_lo) {
            f32x16_t acc[2];
            scores_t<HD>(kl, qf, acc, lane);
            float sv[2][16];
            float mb = -INFINITY;
#pragma unroll
            for (int t = 0; t < 2; ++t)
#pragma unroll
                for (int i = 0; i < 16; ++i) {
                    const int64_t key = key0 + 32 * t + 8 * (i / 4) + 4 * hl + (i % 4);
                    sv[t][i] = allowed(key) ? score(acc[t][i]) : -INFINITY;
                    mb = fmaxf(mb, sv[t][i]);
                }
            mb = fmaxf(mb, __shfl_xor(mb, 32, 64));
            const float mn = fmaxf(m, mb);
            if (mn != -INFINITY) {
                const float alpha = m == -INFINITY ? 0.0f : expf(m - mn);
                float part = 0.0f;
#pragma unroll
                for (int t = 0; t < 2; ++t)
#pragma unroll
                    for (int i = 0; i < 16; ++i) part = part + expf(sv[t][i] - mn);
                lsum = lsum * alpha + part;
                m = mn;
            }
        }
        __syncthreads();
    }
    const float ltot = lsum + __shfl_xor(lsum, 32, 64);

    // ---- pass 2: bf16 probabilities and P V.
    constexpr int NT = HD / 32;
    f32x16_t o[NT];
#pragma unroll
    for (int n = 0; n < NT; ++n) o[n] = f32x16_t{};
    for (int64_t kb = kb_begin; kb < kb_end; ++kb) {
        const int64_t key0 = kb * kBk;
        stage_k<HD>(kl, kbase, kv_stride, key0, T);
        stage_v<HD>(vl, vbase, kv_stride, key0, T);
        __syncthreads();
        if (wave_live && key0 <= wq_last && key0 + kBk > wk_lo) {
            f32x16_t acc[2];
            scores_t<HD>(kl, qf, acc, lane);
#pragma unroll
            for (int t = 0; t < 2; ++t) {
                uint32_t pb[16];
#pragma unroll
                for (int i = 0; i < 16; ++i) {
                    const int64_t key = key0 + 32 * t + 8 * (i / 4) + 4 * hl + (i % 4);
                    const float p = allowed(key) ? expf(score(acc[t][i]) - m) / ltot : 0.0f;
                    pb[i] = bf16_bits_rne(p);
                }
#pragma unroll
                for (int j = 0; j < 2; ++j) {
                    u32x4_t pa;
#pragma unroll
                    for (int e = 0; e < 4; ++e) pa[e] = pb[8 * j + 2 * e] | (pb[8 * j + 2 * e + 1] << 16);
                    const int kofs = (32 * t + 16 * j + 4 * hl) * 2;
#pragma unroll
                    for (int n = 0; n < NT; ++n) {
                        const char* vr = vl + (32 * n + c) * L::VROW + kofs;
                        const u32x2_t v0 = *(const u32x2_t*)vr;
                        const u32x2_t v1 = *(const u32x2_t*)(vr + 16);
                        const u32x4_t vb = {v0[0], v0[1], v1[0], v1[1]};
                        o[n] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
                            __builtin_bit_cast(bf16x8_t, pa), __builtin_bit_cast(bf16x8_t, vb),
                            o[n], 0, 0, 0);
                    }
                }
            }
        }
        __syncthreads();
    }

    // context = round_bf16(sum); D row 8 (i / 4) + 4 hl + i % 4 = query, column = dim.
    if (!wave_live) return;
#pragma unroll
    for (int n = 0; n < NT; ++n)
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const int64_t qrow = qw0 + 8 * (i / 4) + 4 * hl + (i % 4);
            if (qrow >= T) continue;
            const uint32_t bits = bf16_bits_rne(o[n][i]);
            const int64_t off = (b * T + qrow) * out_stride + (int64_t)h * HD + 32 * n + c;
            if (OUT_MODE == NCM_OUT_BF16)
                ((uint16_t*)out)[off] = (uint16_t)bits;
            else
                ((float*)out)[off] = __uint_as_float(bits << 16);
        }
}

template <int HD>
static hipError_t launch_attn_hd(const uint16_t* q, const uint16_t* k, const uint16_t* v,
                                 void* out, int64_t batch, int64_t T, int hq, int hkv,
                                 int64_t q_stride, int64_t kv_stride, int64_t out_stride,
                                 int64_t window, int out_mode, hipStream_t stream) {
    const dim3 grid((unsigned)((T + kBq - 1) / kBq), (unsigned)hq, (unsigned)batch);
    const float scale = 1.0f / sqrtf((float)HD);
    const int group = hq / hkv;
    if (out_mode == NCM_OUT_BF16)
        hipLaunchKernelGGL((attention_bf16_kernel<HD, NCM_OUT_BF16>), grid, dim3(256), 0, stream,
                           q, k, v, out, T, group, q_stride, kv_stride, out_stride, window, scale);
    else
        hipLaunchKernelGGL((attention_bf16_kernel<HD, NCM_OUT_BF16_F32>), grid, dim3(256), 0,
                           stream, q, k, v, out, T, group, q_stride, kv_stride, out_stride, window,
                           scale);
    return hipGetLastError();
}

hipError_t launch_attention_bf16(const uint16_t* q, const uint16_t* k, const uint16_t* v,
                                 void* out, int64_t batch, int64_t seq_len, int q_heads,
                                 int kv_heads, int head_dim, int64_t q_stride, int64_t kv_stride,
                                 int64_t out_stride, int64_t window, int out_mode,
                                 hipStream_t stream) {
    switch (head_dim) {
        case 64:
            return launch_attn_hd<64>(q, k, v, out, batch, seq_len, q_heads, kv_heads, q_stride,
                                      kv_stride, out_stride, window, out_mode, stream);
        case 128:
            return launch_attn_hd<128>(q, k, v, out, batch, seq_len, q_heads, kv_heads, q_stride,
                                       kv_stride, out_stride, window, out_mode, stream);
        default:
            return hipErrorInvalidValue;
    }
}

}  // namespace ncm
