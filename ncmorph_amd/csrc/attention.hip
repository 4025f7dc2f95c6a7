// Causal bf16 attention for the decoder's prefill (packages/kernels/root.zig:
// 536-578, softmax :272-284, mask :380-399), after the q/k/v projections and
// the rotation. Per query and head, in the reference's bf16 mode:
//   s_k = round(round(q . k_k) * 1/sqrt(head_dim))   (k allowed by the mask)
//   p_k = round(exp(s_k - max s) / sum exp(s - max s))
//   context = round(sum_k p_k v_k)
// Every value entering a product is bf16, so q . k and p v are sums of exact
// fp32 products; the MFMA sums them in its own order instead of the
// reference's key order, and the softmax sum is kept online. exp(x) is
// computed as exp2(x log2 e) (v_exp_f32, relative error ~2^-20 at |x| ~ 20)
// and the division as a product with 1 / sum, so a probability can land on
// the other side of a bf16 rounding boundary now and then. Results agree
// with the reference within a few bf16 steps, not bit for bit.
//
// Two passes over the key blocks of one (sequence, head, 128 queries)
// workgroup: pass 1 finds max s and the softmax sum; pass 2 recomputes the
// scores, forms the bf16 probabilities and accumulates P V. Keys are
// processed in blocks of 64: K rows staged in LDS (row-padded), V staged
// transposed (one LDS row per head dimension) so that each lane's eight
// P-operand keys are two 8-byte LDS reads.
//
// Scores are computed transposed, S^T = K Q^T, with v_mfma_f32_32x32x16_bf16,
// one 32-key tile at a time (the running max and sum are updated per tile):
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

// K block [kBk keys][HD] -> registers -> LDS rows; keys at or past `valid`
// are zero. The load for the next block is issued before the current block's
// compute and stored to LDS after it, so its latency overlaps the MFMA work.
template <int HD>
struct KRegs {
    static constexpr int CPR = HD / 8;  // 16-byte chunks per row
    static constexpr int N = kBk * CPR / 256;
    u32x4_t r[N];
};

template <int HD>
__device__ __forceinline__ void load_k(KRegs<HD>& R, const uint16_t* kbase, int64_t kv_stride,
                                       int64_t key0, int64_t valid) {
    constexpr int CPR = KRegs<HD>::CPR;
#pragma unroll
    for (int j = 0; j < KRegs<HD>::N; ++j) {
        const int chunk = threadIdx.x + 256 * j;
        const int row = chunk / CPR, cc = chunk % CPR;
        R.r[j] = u32x4_t{0u, 0u, 0u, 0u};
        if (key0 + row < valid) R.r[j] = *(const u32x4_t*)(kbase + (key0 + row) * kv_stride + 8 * cc);
    }
}

template <int HD>
__device__ __forceinline__ void store_k(char* kl, const KRegs<HD>& R) {
    constexpr int CPR = KRegs<HD>::CPR;
#pragma unroll
    for (int j = 0; j < KRegs<HD>::N; ++j) {
        const int chunk = threadIdx.x + 256 * j;
        const int row = chunk / CPR, cc = chunk % CPR;
        *(u32x4_t*)(kl + row * AttnLds<HD>::KROW + 16 * cc) = R.r[j];
    }
}

// V block [kBk keys][HD] -> LDS V^T [HD][kBk] (keys at or past `valid` zero).
// Task (key pair kp, dim chunk dc): two 16-byte global loads, eight 4-byte
// LDS stores; consecutive threads take consecutive key pairs, so a wave's
// stores to one V^T row are contiguous.
template <int HD>
struct VRegs {
    static constexpr int N = (kBk / 2) * (HD / 8) / 256;
    u32x4_t a[N], b[N];
};

template <int HD>
__device__ __forceinline__ void load_v(VRegs<HD>& R, const uint16_t* vbase, int64_t kv_stride,
                                       int64_t key0, int64_t valid) {
#pragma unroll
    for (int j = 0; j < VRegs<HD>::N; ++j) {
        const int task = threadIdx.x + 256 * j;
        const int kp = task % (kBk / 2), dc = task / (kBk / 2);
        const int64_t k0 = key0 + 2 * kp;
        R.a[j] = u32x4_t{0u, 0u, 0u, 0u};
        R.b[j] = u32x4_t{0u, 0u, 0u, 0u};
        if (k0 < valid) R.a[j] = *(const u32x4_t*)(vbase + k0 * kv_stride + 8 * dc);
        if (k0 + 1 < valid) R.b[j] = *(const u32x4_t*)(vbase + (k0 + 1) * kv_stride + 8 * dc);
    }
}

template <int HD>
__device__ __forceinline__ void store_v(char* vl, const VRegs<HD>& R) {
#pragma unroll
    for (int j = 0; j < VRegs<HD>::N; ++j) {
        const int task = threadIdx.x + 256 * j;
        const int kp = task % (kBk / 2), dc = task / (kBk / 2);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const uint32_t lo = (R.a[j][e] & 0xFFFFu) | (R.b[j][e] << 16);
            const uint32_t hi = (R.a[j][e] >> 16) | (R.b[j][e] & 0xFFFF0000u);
            *(uint32_t*)(vl + (8 * dc + 2 * e) * AttnLds<HD>::VROW + 4 * kp) = lo;
            *(uint32_t*)(vl + (8 * dc + 2 * e + 1) * AttnLds<HD>::VROW + 4 * kp) = hi;
        }
    }
}

// One S^T tile for one wave: keys key0 + 32 t + [0, 32) x its 32 queries.
template <int HD>
__device__ __forceinline__ f32x16_t score_tile(const char* kl, const u32x4_t (&qf)[HD / 16],
                                               int t, int lane) {
    const int c = lane & 31, hl = lane >> 5;
    f32x16_t a = {};
#pragma unroll
    for (int s = 0; s < HD / 16; ++s) {
        const u32x4_t kf =
            *(const u32x4_t*)(kl + (32 * t + c) * AttnLds<HD>::KROW + (16 * s + 8 * hl) * 2);
        a = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, kf),
                                                    __builtin_bit_cast(bf16x8_t, qf[s]), a, 0,
                                                    0, 0);
    }
    return a;
}

__device__ __forceinline__ int wave_min_i(int v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = min(v, __shfl_xor(v, o, 64));
    return v;
}
__device__ __forceinline__ int wave_max_i(int v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = max(v, __shfl_xor(v, o, 64));
    return v;
}

}  // namespace

// Prefix + level-block mask (MASK = 1): key k is allowed for query q when k
// is a prefix key (k < prefix) that is not padded, or k lies in q's own
// range [seg_lo[q], seg_hi[q]) (NCM's block-diagonal mask,
// src/ncm_mask.zig:10-42: prefix queries have an empty range). Positions
// are per sequence. pad: bit (k % 64) of word k / 64 set = prefix key k
// padded; null = none.
struct SegArgs {
    int64_t prefix;
    const int32_t* seg_lo;
    const int32_t* seg_hi;
    const uint64_t* pad;
};

template <int HD, int OUT_MODE, int MASK, bool POW2 = (HD == 64)>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu((HD == 64 || MASK == 1) ? 2 : 1, 4)))
void attention_bf16_kernel(
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ k,
    const uint16_t* __restrict__ v, void* __restrict__ out, int64_t T, int group,
    int64_t q_stride, int64_t kv_stride, int64_t out_stride, int64_t window, float scale,
    SegArgs sa) {
    __shared__ int seg_red[8];
    using L = AttnLds<HD>;
    __shared__ __attribute__((aligned(16))) char kl[L::K_BYTES];
    __shared__ __attribute__((aligned(16))) char vl[L::V_BYTES];

    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int c = lane & 31, hl = lane >> 5;
    const int64_t b = blockIdx.z;
    const int h = blockIdx.y, kvh = h / group;
    // Causal balance: workgroup x takes query block nqb - 1 - x (the most
    // keys) and then block x (the fewest), so every workgroup walks about
    // the same number of key blocks (the middle block of an odd count is
    // taken once).
    // Level mask: one query block per workgroup, the last (longest level)
    // blocks first.
    const int nqb = (int)((T + kBq - 1) / kBq);
    for (int part = 0; part < 2; ++part) {
    const int qbi = part == 0 ? nqb - 1 - (int)blockIdx.x : (int)blockIdx.x;
    if (part == 1 && (MASK == 1 || qbi == nqb - 1 - (int)blockIdx.x)) break;
    const int64_t q0 = (int64_t)qbi * kBq;
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

    const bool wave_live = qw0 < T;
    const int64_t wq_last = (qw0 + 31 < T ? qw0 + 31 : T - 1);
    // The key blocks the workgroup walks: [kb_begin, kb_end) (causal), or
    // the prefix blocks [0, kb_pre) and then the level blocks
    // [kb_seg0, kb_end) (MASK 1); a block outside both is skipped.
    int64_t kb_begin, kb_end, kb_pre = 0, kb_seg0 = 0;
    // Causal: this wave's first visible key. MASK 1: this lane's range and
    // the wave's extremes (w_lo / w_hi: union; w_maxlo / w_minhi: the range
    // every query of the wave sees).
    int64_t wk_lo = 0;
    int seg_lo_q = 0, seg_hi_q = 0, w_lo = 0, w_hi = 0, w_maxlo = 0, w_minhi = 0;
    if (MASK == 0) {
        // Keys <= the workgroup's last query; with a window, keys > (first
        // query - window).
        const int64_t q_last = (q0 + kBq < T ? q0 + kBq : T) - 1;
        int64_t k_lo = window > 0 ? q0 - window + 1 : 0;
        if (k_lo < 0) k_lo = 0;
        kb_begin = k_lo / kBk;
        kb_end = q_last / kBk + 1;
        wk_lo = window > 0 ? qw0 - window + 1 : 0;
        if (wk_lo < 0) wk_lo = 0;
    } else {
        const int P = (int)sa.prefix;
        if (qq < T) {
            seg_lo_q = sa.seg_lo[qq] > P ? sa.seg_lo[qq] : P;
            seg_hi_q = sa.seg_hi[qq] < T ? sa.seg_hi[qq] : (int)T;
            if (seg_hi_q < seg_lo_q) seg_hi_q = seg_lo_q;
        }
        const bool live = qq < T;
        const bool nonempty = live && seg_hi_q > seg_lo_q;
        w_lo = wave_min_i(nonempty ? seg_lo_q : 0x7FFFFFFF);
        w_hi = wave_max_i(nonempty ? seg_hi_q : 0);
        w_maxlo = wave_max_i(live ? seg_lo_q : 0);
        w_minhi = wave_min_i(live ? seg_hi_q : 0x7FFFFFFF);
        __syncthreads();  // the previous part's readers are done with seg_red
        if (lane == 0) { seg_red[2 * wave] = w_lo; seg_red[2 * wave + 1] = w_hi; }
        __syncthreads();
        int g_lo = 0x7FFFFFFF, g_hi = 0;
#pragma unroll
        for (int w = 0; w < 4; ++w) {
            g_lo = min(g_lo, seg_red[2 * w]);
            g_hi = max(g_hi, seg_red[2 * w + 1]);
        }
        kb_pre = (P + kBk - 1) / kBk;
        if (g_hi > g_lo) {
            kb_seg0 = g_lo / kBk;
            kb_end = (g_hi + kBk - 1) / kBk;
            if (kb_end < kb_pre) kb_end = kb_pre;
        } else {
            kb_seg0 = kb_pre;
            kb_end = kb_pre;
        }
        kb_begin = kb_pre > 0 ? 0 : kb_seg0;
    }
    auto next_kb = [&](int64_t kb) {
        if (MASK == 0) return kb + 1;
        ++kb;
        return kb >= kb_pre && kb < kb_seg0 ? kb_seg0 : kb;
    };
    // Whether this wave has any visible key in the block at key0.
    auto wave_sees = [&](int64_t key0) {
        if (!wave_live) return false;
        if (MASK == 0) return key0 <= wq_last && key0 + kBk > wk_lo;
        return key0 < sa.prefix || (key0 + kBk > w_lo && key0 < w_hi);
    };
    // Padded-prefix bits of the block at key0 (MASK 1).
    auto pad_bits = [&](int64_t key0) -> uint64_t {
        return (MASK == 1 && sa.pad && key0 < sa.prefix) ? sa.pad[key0 / kBk] : 0ull;
    };
    // A block is "full" for this wave when every key in it is allowed for
    // all 32 of its queries: only blocks on the diagonal or a window's or
    // range's edge need the per-element test.
    auto block_full = [&](int64_t key0) {
        if (MASK == 0)
            return key0 + kBk - 1 <= qw0 && key0 + kBk <= T &&
                   (window <= 0 || key0 + window > qw0 + 31);
        return (key0 + kBk <= sa.prefix && pad_bits(key0) == 0) ||
               (key0 >= sa.prefix && key0 >= w_maxlo && key0 + kBk <= w_minhi &&
                wq_last == qw0 + 31);
    };
    const int koff = 4 * hl;  // + 32 t + 8 (i / 4) + i % 4: the key of element i of tile t
    // bf16 RNE without the NaN canonicalisation of bf16_bits_rne: exact for
    // every finite or infinite value (scores and probabilities here; a NaN
    // input propagates as some NaN or garbage, where the reference's whole
    // row is NaN).
    auto rnd = [](float x) {
        const uint32_t u = __float_as_uint(x);
        return __uint_as_float((u + 0x7FFFu + ((u >> 16) & 1u)) & 0xFFFF0000u);
    };
    auto score = [&](float acc) { return rnd(rnd(acc) * scale); };
    // The scores of a whole tile, two per v_cvt_pk_bf16_f32 (the same bits
    // as rnd / score for every non-NaN value).
    auto round_pairs = [](f32x16_t& v) {
#pragma unroll
        for (int i = 0; i < 16; i += 2) {
            const uint32_t p = bf16x2_rne(v[i], v[i + 1]);
            v[i] = __uint_as_float(p << 16);
            v[i + 1] = __uint_as_float(p & 0xFFFF0000u);
        }
    };
    auto to_scores = [&](f32x16_t& v) {
        round_pairs(v);
        if (!POW2) {
#pragma unroll
            for (int i = 0; i < 16; ++i) v[i] = v[i] * scale;
            round_pairs(v);
        }
    };
    // exp(s - m) as exp2(s log2 e - m log2 e): v_exp_f32 on one FMA.
    constexpr float kLog2e = 1.4426950408889634f;
    // The exp2 argument of a raw sum: fma(score, log2 e, -m log2 e). When the
    // scale is a power of two (head_dim 64: 1/8), round(acc) * scale is exact
    // and already a bf16 value, so the second rounding is the identity and
    // the scale folds into the FMA's multiplier without changing its result
    // (round(acc) * (scale log2e) is the same real product as score * log2e).
    // The one exception, a product below 2^-126, moves the FMA's addend by
    // less than 2^-130 and cannot change exp2 of the sum.
    const float sl = POW2 ? scale * kLog2e : kLog2e;
    // s: a tile value after to_scores (for POW2 the rounded sum; the scale
    // sits in sl).
    auto expo = [&](float s, float nm_) { return fmaf(s, sl, nm_); };
    // Per-element mask inside a block: key offset kr (element i of tile t) is
    // allowed for query offset rq when kr <= rq, kr < rt (keys before T) and
    // kr > rw (inside the window).
    auto kr_of = [&](int t, int i) { return 32 * t + 8 * (i / 4) + (i % 4) + koff; };

    // ---- pass 1: running max and softmax sum per query. score() is
    // monotone in the accumulated dot product, so the block maximum is taken
    // on the raw sums and scored once.
    float m = -INFINITY, lsum = 0.0f;
    KRegs<HD> kr;
    load_k<HD>(kr, kbase, kv_stride, kb_begin * kBk, T);
    for (int64_t kb = kb_begin; kb < kb_end; kb = next_kb(kb)) {
        const int64_t key0 = kb * kBk;
        const int64_t kb_next = next_kb(kb);
        store_k<HD>(kl, kr);
        lds_barrier();
        if (kb_next < kb_end) load_k<HD>(kr, kbase, kv_stride, kb_next * kBk, T);
        if (wave_sees(key0)) {
            const bool full = block_full(key0);
            // Causal: key offset kr is allowed when kr <= rq, kr < rt (keys
            // before T) and kr > rw (inside the window). MASK 1: kr < rp is a
            // prefix key (allowed unless its pad bit is set), else allowed
            // when rlo <= kr < rhi (offsets clamped to [-1, kBk]).
            const int rq = (int)(qq - key0), rt = (int)(T - key0 < kBk ? T - key0 : kBk);
            const int rw = window > 0 ? (int)(rq - window) : -(1 << 30);
            auto clampk = [](int64_t x) { return (int)(x < -1 ? -1 : (x > kBk ? kBk : x)); };
            const int rp = MASK == 1 ? clampk(sa.prefix - key0) : 0;
            const int rlo = MASK == 1 ? clampk(seg_lo_q - key0) : 0;
            const int rhi = MASK == 1 ? clampk(seg_hi_q - key0) : 0;
            const uint64_t pbits = pad_bits(key0);
            auto ok = [&](int kk) {
                if (MASK == 0) return kk <= rq && kk < rt && kk > rw;
                return kk < rp ? ((pbits >> kk) & 1ull) == 0ull : (kk >= rlo && kk < rhi);
            };
#pragma unroll
            for (int t = 0; t < 2; ++t) {
                f32x16_t acc = score_tile<HD>(kl, qf, t, lane);
                if (!full)
#pragma unroll
                    for (int i = 0; i < 16; ++i) {
                        const int k = kr_of(t, i);
                        acc[i] = ok(k) ? acc[i] : -INFINITY;
                    }
                float mb = -INFINITY;
#pragma unroll
                for (int i = 0; i < 16; ++i) mb = fmaxf(mb, acc[i]);
                mb = fmaxf(mb, __shfl_xor(mb, 32, 64));
                mb = POW2 ? rnd(mb) * scale : score(mb);
                const float mn = fmaxf(m, mb);
                if (mn != -INFINITY) {
                    const float nm = -mn * kLog2e;
                    const float alpha =
                        m == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(fmaf(m, kLog2e, nm));
                    to_scores(acc);
                    float part = 0.0f;
#pragma unroll
                    for (int i = 0; i < 16; ++i)
                        part = part + __builtin_amdgcn_exp2f(expo(acc[i], nm));
                    lsum = fmaf(lsum, alpha, part);
                    m = mn;
                }
            }
        }
        lds_barrier();
    }
    const float ltot = lsum + __shfl_xor(lsum, 32, 64);
    // A query with no allowed key (a prefix query whose prefix is all
    // padding) gets zero probabilities, hence a zero context, as the
    // reference (root.zig:563-565).
    const bool any_key = ltot > 0.0f;
    const float inv_l = any_key ? 1.0f / ltot : 0.0f;
    const float nm = any_key ? -m * kLog2e : 0.0f;  // m is a score: -m log2 e as in pass 1

    // ---- pass 2: bf16 probabilities and P V.
    constexpr int NT = HD / 32;
    f32x16_t o[NT];
#pragma unroll
    for (int n = 0; n < NT; ++n) o[n] = f32x16_t{};
    VRegs<HD> vr;
    load_k<HD>(kr, kbase, kv_stride, kb_begin * kBk, T);
    load_v<HD>(vr, vbase, kv_stride, kb_begin * kBk, T);
    for (int64_t kb = kb_begin; kb < kb_end; kb = next_kb(kb)) {
        const int64_t key0 = kb * kBk;
        const int64_t kb_next = next_kb(kb);
        store_k<HD>(kl, kr);
        store_v<HD>(vl, vr);
        lds_barrier();
        if (kb_next < kb_end) {
            load_k<HD>(kr, kbase, kv_stride, kb_next * kBk, T);
            load_v<HD>(vr, vbase, kv_stride, kb_next * kBk, T);
        }
        if (wave_sees(key0)) {
            const bool full = block_full(key0);
            // Causal: key offset kr is allowed when kr <= rq, kr < rt (keys
            // before T) and kr > rw (inside the window). MASK 1: kr < rp is a
            // prefix key (allowed unless its pad bit is set), else allowed
            // when rlo <= kr < rhi (offsets clamped to [-1, kBk]).
            const int rq = (int)(qq - key0), rt = (int)(T - key0 < kBk ? T - key0 : kBk);
            const int rw = window > 0 ? (int)(rq - window) : -(1 << 30);
            auto clampk = [](int64_t x) { return (int)(x < -1 ? -1 : (x > kBk ? kBk : x)); };
            const int rp = MASK == 1 ? clampk(sa.prefix - key0) : 0;
            const int rlo = MASK == 1 ? clampk(seg_lo_q - key0) : 0;
            const int rhi = MASK == 1 ? clampk(seg_hi_q - key0) : 0;
            const uint64_t pbits = pad_bits(key0);
            auto ok = [&](int kk) {
                if (MASK == 0) return kk <= rq && kk < rt && kk > rw;
                return kk < rp ? ((pbits >> kk) & 1ull) == 0ull : (kk >= rlo && kk < rhi);
            };
#pragma unroll
            for (int t = 0; t < 2; ++t) {
                f32x16_t acc = score_tile<HD>(kl, qf, t, lane);
                if (!full)
#pragma unroll
                    for (int i = 0; i < 16; ++i) {
                        const int k = kr_of(t, i);
                        acc[i] = ok(k) ? acc[i] : -INFINITY;
                    }
                // p = round_bf16(e / sum), packed two per register.
                to_scores(acc);
                float pf[16];
#pragma unroll
                for (int i = 0; i < 16; ++i)
                    pf[i] = __builtin_amdgcn_exp2f(expo(acc[i], nm)) * inv_l;
#pragma unroll
                for (int j = 0; j < 2; ++j) {
                    u32x4_t pa;
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        pa[e] = bf16x2_rne(pf[8 * j + 2 * e], pf[8 * j + 2 * e + 1]);
                    const int kofs = (32 * t + 16 * j + 4 * hl) * 2;
#pragma unroll
                    for (int n = 0; n < NT; ++n) {
                        const char* vp = vl + (32 * n + c) * L::VROW + kofs;
                        const u32x2_t v0 = *(const u32x2_t*)vp;
                        const u32x2_t v1 = *(const u32x2_t*)(vp + 16);
                        const u32x4_t vb = {v0[0], v0[1], v1[0], v1[1]};
                        o[n] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
                            __builtin_bit_cast(bf16x8_t, pa), __builtin_bit_cast(bf16x8_t, vb),
                            o[n], 0, 0, 0);
                    }
                }
            }
        }
        lds_barrier();
    }

    // context = round_bf16(sum); D row 8 (i / 4) + 4 hl + i % 4 = query, column = dim.
    if (wave_live) {
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
    }  // part
}

template <int HD, int MASK>
static hipError_t launch_attn_hd(const uint16_t* q, const uint16_t* k, const uint16_t* v,
                                 void* out, int64_t batch, int64_t T, int hq, int hkv,
                                 int64_t q_stride, int64_t kv_stride, int64_t out_stride,
                                 int64_t window, SegArgs sa, int out_mode, hipStream_t stream) {
    const int64_t nqb = (T + kBq - 1) / kBq;
    const dim3 grid((unsigned)(MASK == 0 ? (nqb + 1) / 2 : nqb), (unsigned)hq, (unsigned)batch);
    const float scale = 1.0f / sqrtf((float)HD);
    const int group = hq / hkv;
    if (out_mode == NCM_OUT_BF16)
        hipLaunchKernelGGL((attention_bf16_kernel<HD, NCM_OUT_BF16, MASK>), grid, dim3(256), 0,
                           stream, q, k, v, out, T, group, q_stride, kv_stride, out_stride, window,
                           scale, sa);
    else
        hipLaunchKernelGGL((attention_bf16_kernel<HD, NCM_OUT_BF16_F32, MASK>), grid, dim3(256),
                           0, stream, q, k, v, out, T, group, q_stride, kv_stride, out_stride,
                           window, scale, sa);
    return hipGetLastError();
}

hipError_t launch_attention_bf16(const uint16_t* q, const uint16_t* k, const uint16_t* v,
                                 void* out, int64_t batch, int64_t seq_len, int q_heads,
                                 int kv_heads, int head_dim, int64_t q_stride, int64_t kv_stride,
                                 int64_t out_stride, int64_t window, int out_mode,
                                 hipStream_t stream) {
    // A window of seq_len or more admits every causal key.
    if (window >= seq_len) window = 0;
    const SegArgs none{0, nullptr, nullptr, nullptr};
    switch (head_dim) {
        case 64:
            return launch_attn_hd<64, 0>(q, k, v, out, batch, seq_len, q_heads, kv_heads, q_stride,
                                         kv_stride, out_stride, window, none, out_mode, stream);
        case 128:
            return launch_attn_hd<128, 0>(q, k, v, out, batch, seq_len, q_heads, kv_heads,
                                          q_stride, kv_stride, out_stride, window, none, out_mode,
                                          stream);
        default:
            return hipErrorInvalidValue;
    }
}

hipError_t launch_attention_bf16_seg(const uint16_t* q, const uint16_t* k, const uint16_t* v,
                                     void* out, int64_t batch, int64_t seq_len, int q_heads,
                                     int kv_heads, int head_dim, int64_t q_stride,
                                     int64_t kv_stride, int64_t out_stride, int64_t prefix,
                                     const int32_t* seg_lo, const int32_t* seg_hi,
                                     const uint64_t* pad, int out_mode, hipStream_t stream) {
    const SegArgs sa{prefix, seg_lo, seg_hi, pad};
    switch (head_dim) {
        case 64:
            return launch_attn_hd<64, 1>(q, k, v, out, batch, seq_len, q_heads, kv_heads, q_stride,
                                         kv_stride, out_stride, 0, sa, out_mode, stream);
        case 128:
            return launch_attn_hd<128, 1>(q, k, v, out, batch, seq_len, q_heads, kv_heads,
                                          q_stride, kv_stride, out_stride, 0, sa, out_mode,
                                          stream);
        default:
            return hipErrorInvalidValue;
    }
}

}  // namespace ncm
