// bf16 attention after the q/k/v projections and the rotation
// (packages/kernels/root.zig:536-578, softmax :272-284, causal mask
// :380-399), causal or with NCM's prefix + level mask. Per query and head, in
// the reference's bf16 mode:
//   s_k = round(round(q . k_k) * 1/sqrt(head_dim))   (k allowed by the mask)
//   p_k = round(exp(s_k - max s) / sum exp(s - max s))
//   context = round(sum_k p_k v_k)
// Every value entering a product is bf16, so q . k and p v are sums of exact
// fp32 products; the MFMA sums them in its own order instead of the
// reference's key order, and the softmax sum is kept online. exp(x) is
// computed as exp2(x log2 e) (v_exp_f32, relative error ~2^-20 at |x| ~ 20)
// and the division by the sum as a term - log2(sum) of the same exponent
// (v_log_f32), so a probability can land on the other side of a bf16
// rounding boundary now and then. Results agree
// with the reference within a few bf16 steps, not bit for bit.
//
// Two passes over the key blocks of one (sequence, head, 32 NWV queries)
// workgroup of NWV wavefronts (32 queries each): pass 1 finds max s and the
// softmax sum; pass 2 recomputes the scores, forms the bf16 probabilities and
// accumulates P V. The probabilities need the final sum before they are
// rounded, hence the two passes. Keys are processed in blocks of 64, loaded
// global -> LDS directly (buffer loads into LDS, two stages: the next block's
// loads fly while the current block is computed, one barrier per block):
// K rows as stored, and V from a transposed copy V^T [batch][kv head][dim]
// [keys, padded to 64] that attention_vt_kernel writes first. LDS rows keep
// 16-byte chunks XOR-swizzled by row so that the fragment reads of 16
// consecutive rows hit 16 distinct bank groups.
//
// Scores are computed transposed, S^T = K Q^T, with v_mfma_f32_32x32x16_bf16,
// one 32-key tile at a time (the running max and sum are updated per tile).
// The A operand's row m of a tile is key perm(m), perm swapping bits 2 and 3
// of m; lane l then holds query l % 32 and key perm(8 (i / 4) + 4 (l / 32) +
// i % 4) in element i, which for elements 8j .. 8j+7 is keys 16j + 8 (l / 32)
// .. + 7: exactly the A operand of P V for the k-step of keys 16j .. 16j + 15,
// whose B operand (8 consecutive keys of one dim per lane) is then one
// 16-byte chunk of a V^T row.
#include "common.h"
#include "gemm_core.h"
#include "linear.h"

namespace ncm {

namespace {

constexpr int kBk = 64;  // keys per block

// LDS layout of one stage: the K block [kBk keys][HD] (rows of 2 HD bytes)
// then the V^T block [HD dims][kBk keys] (rows of 128 bytes); chunk c of row
// r sits in slot c ^ ((r >> SWZ) & (CH - 1)). A direct-to-LDS instruction
// fills 1 KB: RPI consecutive rows.
template <int HD, int NWV>
struct AttnTile {
    static constexpr int KRB = 2 * HD;
    static constexpr int KCH = KRB / 16;
    static constexpr int KSWZ = KRB == 256 ? 0 : 1;
    static constexpr int KRPI = 1024 / KRB;
    static constexpr int K_BYTES = kBk * KRB;
    static constexpr int K_DMA = kBk / KRPI / NWV;  // K instructions per wavefront
    static constexpr int VRB = 2 * kBk;
    static constexpr int VCH = VRB / 16;
    static constexpr int VSWZ = 1;
    static constexpr int VRPI = 1024 / VRB;
    static constexpr int V_BYTES = HD * VRB;
    static constexpr int V_DMA = HD / VRPI / NWV;
    static constexpr int STAGE = K_BYTES + V_BYTES;
    static constexpr int LDS = 2 * STAGE;
    static_assert(K_DMA >= 1 && K_DMA * KRPI * NWV == kBk, "K loader shape");
    static_assert(V_DMA >= 1 && V_DMA * VRPI * NWV == HD, "V loader shape");
    static_assert(LDS <= 64 * 1024, "at least two workgroups per CU");
};

// Row m of a 32-key score tile holds key perm(m): bits 2 and 3 swapped.
__device__ __forceinline__ int key_perm(int m) {
    return (m & ~0xC) | ((m & 4) << 1) | ((m & 8) >> 1);
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

// V [batch * T rows, row stride kv_stride, head h at column h * HD] ->
// V^T [batch][kv_heads][HD][Tp] (Tp = T rounded up to kBk, keys >= T zero),
// through 64 x 64 LDS tiles. Grid: (Tp / 64, kv_heads * HD / 64, batch).
__global__ __launch_bounds__(256) void attention_vt_kernel(const uint16_t* __restrict__ v,
                                                           uint16_t* __restrict__ vt, int64_t T,
                                                           int64_t Tp, int64_t kv_stride,
                                                           int64_t kv_width) {
    __shared__ uint16_t tile[64][64 + 8];
    const int64_t key0 = (int64_t)blockIdx.x * 64;
    const int64_t col0 = (int64_t)blockIdx.y * 64;  // column in [0, kv_heads * HD)
    const int64_t b = blockIdx.z;
    const int tid = threadIdx.x;
    // Load: thread t takes key key0 + (t / 8) + 32 p, columns col0 + 8 (t % 8) .. + 7.
#pragma unroll
    for (int p = 0; p < 2; ++p) {
        const int kr = tid / 8 + 32 * p, cc = 8 * (tid % 8);
        u32x4_t x = {0u, 0u, 0u, 0u};
        if (key0 + kr < T) x = *(const u32x4_t*)(v + (b * T + key0 + kr) * kv_stride + col0 + cc);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            tile[kr][cc + 2 * e] = (uint16_t)(x[e] & 0xFFFFu);
            tile[kr][cc + 2 * e + 1] = (uint16_t)(x[e] >> 16);
        }
    }
    __syncthreads();
    // Store: thread t takes column col0 + (t / 8) + 32 p, keys key0 + 8 (t % 8) .. + 7.
#pragma unroll
    for (int p = 0; p < 2; ++p) {
        const int c = tid / 8 + 32 * p, k8 = 8 * (tid % 8);
        u32x4_t o;
#pragma unroll
        for (int e = 0; e < 4; ++e)
            o[e] = (uint32_t)tile[k8 + 2 * e][c] | ((uint32_t)tile[k8 + 2 * e + 1][c] << 16);
        *(u32x4_t*)(vt + (b * kv_width + col0 + c) * Tp + key0 + k8) = o;
    }
}

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

// The K / V^T stages of the head_dim-128 kernels are dynamic shared memory
// (the launch passes their size): measured 8% faster at NCM's block-diagonal
// level attention and 4% at the block-causal one than the same kernel with
// a static array, with bit-identical results; head_dim 64 keeps the static
// array (1-2% faster there).
template <int HD>
constexpr bool attn_dyn_lds() { return HD == 128; }

template <int HD, int OUT_MODE, int MASK, int NWV, bool POW2 = (HD == 64)>
__global__ __launch_bounds__(64 * NWV)
__attribute__((amdgpu_waves_per_eu(2, 4))) void attention_bf16_kernel(
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ k,
    const uint16_t* __restrict__ vt, void* __restrict__ out, int64_t T, int64_t Tp, int group,
    int kv_heads, int64_t q_stride, int64_t kv_stride, int64_t out_stride, int64_t window,
    float scale, SegArgs sa, int n_xb) {
    using L = AttnTile<HD, NWV>;
    constexpr int kBq = 32 * NWV;  // queries per workgroup
    __shared__ int seg_red[2 * NWV];
    char* lds;
    if constexpr (attn_dyn_lds<HD>()) {
        extern __shared__ __attribute__((aligned(1024))) char lds_dyn[];
        lds = lds_dyn;
    } else {
        __shared__ __attribute__((aligned(1024))) char lds_static[L::LDS];
        lds = lds_static;
    }

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int c = lane & 31, hl = lane >> 5;
    // Workgroup -> (sequence b, kv head, query block xb, head hg of the kv
    // head's group), the kv head slowest but for the sequence and the group's
    // heads fastest: with the XCD remap, each XCD walks a contiguous run of
    // this order, so the K and V^T blocks it streams belong to few kv heads
    // (one per XCD for 8 kv heads and one sequence) and the group's heads read
    // the same blocks at about the same time, from the XCD's L2.
    const int logical = xcd_remap((int)blockIdx.x, (int)gridDim.x);
    const int hg = logical % group;
    const int xb = (logical / group) % n_xb;
    const int kvh = (logical / group / n_xb) % kv_heads;
    const int64_t b = logical / group / n_xb / kv_heads;
    const int h = kvh * group + hg;

    // K rows of this (sequence, kv head): keys >= T load as zero (out of the
    // resource's range). V^T rows: Tp keys each, zero past T.
    const uint16_t* kbase = k + b * T * kv_stride + (int64_t)kvh * HD;
    const __amdgpu_buffer_rsrc_t rsk =
        make_rsrc(kbase, (uint32_t)(((T - 1) * kv_stride + HD) * 2));
    const uint16_t* vbase = vt + ((b * kv_heads + kvh) * HD) * Tp;
    const __amdgpu_buffer_rsrc_t rsv = make_rsrc(vbase, (uint32_t)(HD * Tp * 2));

    // Direct-to-LDS loads of block kb into stage st: wave w's instruction p
    // fills 1 KB of rows; lane l takes row (p NWV + w) RPI + l / CH, slot
    // l % CH, i.e. global chunk slot ^ swizzle(row).
    auto load_k = [&](int st, int64_t kb) {
        char* dst0 = lds + st * L::STAGE;
#pragma unroll
        for (int p = 0; p < L::K_DMA; ++p) {
            const int ins = p * NWV + wave;
            const int row = ins * L::KRPI + lane / L::KCH;
            const int ch = (lane % L::KCH) ^ ((row >> L::KSWZ) & (L::KCH - 1));
            const uint32_t off = (uint32_t)((kb * kBk + row) * kv_stride * 2 + ch * 16);
            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                rsk, (__attribute__((address_space(3))) void*)(dst0 + ins * 1024), 16, off, 0, 0,
                0);
        }
    };
    auto load_v = [&](int st, int64_t kb) {
        char* dst0 = lds + st * L::STAGE + L::K_BYTES;
#pragma unroll
        for (int p = 0; p < L::V_DMA; ++p) {
            const int ins = p * NWV + wave;
            const int row = ins * L::VRPI + lane / L::VCH;
            const int ch = (lane % L::VCH) ^ ((row >> L::VSWZ) & (L::VCH - 1));
            const uint32_t off = (uint32_t)((row * Tp + kb * kBk) * 2 + ch * 16);
            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                rsv, (__attribute__((address_space(3))) void*)(dst0 + ins * 1024), 16, off, 0, 0,
                0);
        }
    };
    // Lane-constant parts of the fragment addresses: K row perm(c) of a tile
    // (its swizzle term), V^T row c of a 32-dim block.
    const int krow = key_perm(c);
    const int kswz = (krow >> L::KSWZ) & (L::KCH - 1);
    const int vswz = (c >> L::VSWZ) & (L::VCH - 1);
    // S^T tile t (keys 32 t .. + 31 of the block) x the wave's 32 queries.
    auto score_tile = [&](const char* kl, const u32x4_t (&qf)[HD / 16], int t) {
        f32x16_t a = {};
        const char* rowp = kl + (32 * t + krow) * L::KRB;
#pragma unroll
        for (int s = 0; s < HD / 16; ++s) {
            const u32x4_t kf = *(const u32x4_t*)(rowp + (((2 * s + hl) ^ kswz) * 16));
            a = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, kf),
                                                        __builtin_bit_cast(bf16x8_t, qf[s]), a,
                                                        0, 0, 0);
        }
        return a;
    };

    // Causal balance: workgroup x takes query block nqb - 1 - x (the most
    // keys) and then block x (the fewest), so every workgroup walks about
    // the same number of key blocks (the middle block of an odd count is
    // taken once). Level mask: one query block per workgroup, the last
    // (longest level) blocks first.
    const int nqb = (int)((T + kBq - 1) / kBq);
    for (int part = 0; part < 2; ++part) {
    const int qbi = part == 0 ? nqb - 1 - xb : xb;
    if (part == 1 && (MASK == 1 || qbi == nqb - 1 - xb)) break;
    const int64_t q0 = (int64_t)qbi * kBq;
    const int64_t qw0 = q0 + 32 * wave;
    const int64_t qq = qw0 + c;  // the query of this lane's score column

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
        for (int w = 0; w < NWV; ++w) {
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
    // The key offset in its block of element i of score tile t.
    auto kr_of = [&](int t, int i) { return 32 * t + key_perm(8 * (i / 4) + 4 * hl + (i % 4)); };
    // Per-element mask inside a block. Causal: key offset kk is allowed when
    // kk <= rq, kk < rt (keys before T) and kk > rw (inside the window).
    // MASK 1: kk < rp is a prefix key (allowed unless its pad bit is set),
    // else allowed when rlo <= kk < rhi (offsets clamped to [-1, kBk]).
    auto apply_mask = [&](f32x16_t& acc, int64_t key0, int t) {
        const int rq = (int)(qq - key0), rt = (int)(T - key0 < kBk ? T - key0 : kBk);
        const int rw = window > 0 ? (int)(rq - window) : -(1 << 30);
        auto clampk = [](int64_t x) { return (int)(x < -1 ? -1 : (x > kBk ? kBk : x)); };
        const int rp = MASK == 1 ? clampk(sa.prefix - key0) : 0;
        const int rlo = MASK == 1 ? clampk(seg_lo_q - key0) : 0;
        const int rhi = MASK == 1 ? clampk(seg_hi_q - key0) : 0;
        const uint64_t pbits = pad_bits(key0);
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const int kk = kr_of(t, i);
            bool ok;
            if (MASK == 0)
                ok = kk <= rq && kk < rt && kk > rw;
            else
                ok = kk < rp ? ((pbits >> kk) & 1ull) == 0ull : (kk >= rlo && kk < rhi);
            acc[i] = ok ? acc[i] : -INFINITY;
        }
    };

    // ---- pass 1: running max and softmax sum per query. score() is
    // monotone in the accumulated dot product, so the block maximum is taken
    // on the raw sums and scored once.
    float m = -INFINITY, lsum = 0.0f;
    __syncthreads();  // the previous part has finished reading both stages
    load_k(0, kb_begin);
    int cur = 0;
    for (int64_t kb = kb_begin; kb < kb_end; kb = next_kb(kb)) {
        const int64_t key0 = kb * kBk;
        const int64_t kb_next = next_kb(kb);
        wait_barrier<0>();  // block kb has landed; stage cur ^ 1 is free
        if (kb_next < kb_end) load_k(cur ^ 1, kb_next);
        const char* kl = lds + cur * L::STAGE;
        if (wave_sees(key0)) {
            const bool full = block_full(key0);
            // Both tiles' scores first: the second tile's MFMAs run while
            // the first tile's softmax work issues.
            f32x16_t accs[2];
#pragma unroll
            for (int t = 0; t < 2; ++t) accs[t] = score_tile(kl, qf, t);
#pragma unroll
            for (int t = 0; t < 2; ++t) {
                f32x16_t& acc = accs[t];
                if (!full) apply_mask(acc, key0, t);
                float mb = -INFINITY;
#pragma unroll
                for (int i = 0; i < 16; ++i) mb = fmaxf(mb, acc[i]);
                {
                    // Max with the other half-wave's value (the same 32 keys'
                    // other 16 rows): a VALU lane swap, no LDS round trip.
                    const u32x2_t sw = swap32(__float_as_uint(mb));
                    mb = fmaxf(__uint_as_float(sw[0]), __uint_as_float(sw[1]));
                }
                mb = POW2 ? rnd(mb) * scale : score(mb);
                const float mn = fmaxf(m, mb);
                if (mn != -INFINITY) {
                    const float nm = -mn * kLog2e;
                    const float alpha =
                        m == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(fmaf(m, kLog2e, nm));
                    to_scores(acc);
                    float part_sum = 0.0f;
#pragma unroll
                    for (int i = 0; i < 16; ++i)
                        part_sum = part_sum + __builtin_amdgcn_exp2f(expo(acc[i], nm));
                    lsum = fmaf(lsum, alpha, part_sum);
                    m = mn;
                }
            }
        }
        cur ^= 1;
    }
    float ltot;
    {
        // lsum plus the other half-wave's lsum (the same sum in both
        // halves: the add commutes).
        const u32x2_t sw = swap32(__float_as_uint(lsum));
        ltot = __uint_as_float(sw[0]) + __uint_as_float(sw[1]);
    }
    // A query with no allowed key (a prefix query whose prefix is all
    // padding) gets zero probabilities, hence a zero context, as the
    // reference (root.zig:563-565).
    // p = exp2(s log2 e - m log2 e - log2 sum): the division by the sum
    // folded into the exponent (no product per score); -inf gives p = 0.
    const bool any_key = ltot > 0.0f;
    const float nm = any_key ? -m * kLog2e - __builtin_amdgcn_logf(ltot) : -INFINITY;

    // ---- pass 2: bf16 probabilities and P V.
    constexpr int NT = HD / 32;
    f32x16_t o[NT];
#pragma unroll
    for (int n = 0; n < NT; ++n) o[n] = f32x16_t{};
    __syncthreads();  // pass 1 has finished reading both stages
    load_k(0, kb_begin);
    load_v(0, kb_begin);
    cur = 0;
    for (int64_t kb = kb_begin; kb < kb_end; kb = next_kb(kb)) {
        const int64_t key0 = kb * kBk;
        const int64_t kb_next = next_kb(kb);
        wait_barrier<0>();
        if (kb_next < kb_end) {
            load_k(cur ^ 1, kb_next);
            load_v(cur ^ 1, kb_next);
        }
        const char* kl = lds + cur * L::STAGE;
        const char* vl = kl + L::K_BYTES;
        if (wave_sees(key0)) {
            const bool full = block_full(key0);
            f32x16_t accs[2];
#pragma unroll
            for (int t = 0; t < 2; ++t) accs[t] = score_tile(kl, qf, t);
#pragma unroll
            for (int t = 0; t < 2; ++t) {
                f32x16_t& acc = accs[t];
                if (!full) apply_mask(acc, key0, t);
                // p = round_bf16(e / sum), packed two per register.
                to_scores(acc);
                float pf[16];
#pragma unroll
                for (int i = 0; i < 16; ++i)
                    pf[i] = __builtin_amdgcn_exp2f(expo(acc[i], nm));
#pragma unroll
                for (int j = 0; j < 2; ++j) {
                    u32x4_t pa;
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        pa[e] = bf16x2_rne(pf[8 * j + 2 * e], pf[8 * j + 2 * e + 1]);
                    // V^T rows 32 n + c, keys 32 t + 16 j + 8 hl .. + 7: chunk 4 t + 2 j + hl.
                    const int vslot = (4 * t + 2 * j + hl) ^ vswz;
#pragma unroll
                    for (int n = 0; n < NT; ++n) {
                        const u32x4_t vb =
                            *(const u32x4_t*)(vl + (32 * n + c) * L::VRB + vslot * 16);
                        o[n] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
                            __builtin_bit_cast(bf16x8_t, pa), __builtin_bit_cast(bf16x8_t, vb),
                            o[n], 0, 0, 0);
                    }
                }
            }
        }
        cur ^= 1;
    }
    // No load may still be writing LDS when the workgroup ends (a walk with
    // no key block issued its first loads and never waited for them).
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt(waitcnt_vm_lgkm0(0));
    asm volatile("" ::: "memory");

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

int64_t attention_vt_padded(int64_t seq_len) { return (seq_len + kBk - 1) / kBk * kBk; }

size_t attention_workspace_bytes(int64_t batch, int64_t seq_len, int kv_heads, int head_dim) {
    return (size_t)batch * kv_heads * head_dim * attention_vt_padded(seq_len) * 2;
}

namespace {

// Waves per workgroup (measured at the decoder's 4 x 1024 causal prefill and
// NCM's 8224-position level attention): 2 for head_dim 64, 4 for head_dim
// 128. Both kernels hold about 200 VGPRs (two wavefronts per SIMD); small
// workgroups keep the per-block barrier short.
template <int HD>
constexpr int attn_waves() { return HD == 64 ? 2 : 4; }

template <int HD, int MASK>
hipError_t launch_attn_hd(const uint16_t* q, const uint16_t* k, const uint16_t* v, void* out,
                          int64_t batch, int64_t T, int hq, int hkv, int64_t q_stride,
                          int64_t kv_stride, int64_t out_stride, int64_t window, SegArgs sa,
                          int out_mode, uint16_t* vt, hipStream_t stream) {
    constexpr int NWV = attn_waves<HD>();
    const int64_t Tp = attention_vt_padded(T);
    hipLaunchKernelGGL(attention_vt_kernel,
                       dim3((unsigned)(Tp / 64), (unsigned)(hkv * HD / 64), (unsigned)batch),
                       dim3(256), 0, stream, v, vt, T, Tp, kv_stride, (int64_t)hkv * HD);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    const int64_t nqb = (T + 32 * NWV - 1) / (32 * NWV);
    const int n_xb = (int)(MASK == 0 ? (nqb + 1) / 2 : nqb);
    const dim3 grid((unsigned)((int64_t)n_xb * hq * batch));
    const float scale = 1.0f / sqrtf((float)HD);
    const int group = hq / hkv;
    auto kb16 = attention_bf16_kernel<HD, NCM_OUT_BF16, MASK, NWV>;
    auto kf32 = attention_bf16_kernel<HD, NCM_OUT_BF16_F32, MASK, NWV>;
    size_t shm = 0;
    if constexpr (attn_dyn_lds<HD>()) {
        shm = AttnTile<HD, NWV>::LDS;
        static const hipError_t attr = [&] {
            hipError_t r = hipFuncSetAttribute((const void*)kb16,
                                               hipFuncAttributeMaxDynamicSharedMemorySize,
                                               (int)AttnTile<HD, NWV>::LDS);
            if (r == hipSuccess)
                r = hipFuncSetAttribute((const void*)kf32,
                                        hipFuncAttributeMaxDynamicSharedMemorySize,
                                        (int)AttnTile<HD, NWV>::LDS);
            return r;
        }();
        if (attr != hipSuccess) return attr;
    }
    if (out_mode == NCM_OUT_BF16)
        hipLaunchKernelGGL(kb16, grid, dim3(64 * NWV), shm, stream, q, k, vt, out, T, Tp, group,
                           hkv, q_stride, kv_stride, out_stride, window, scale, sa, n_xb);
    else
        hipLaunchKernelGGL(kf32, grid, dim3(64 * NWV), shm, stream, q, k, vt, out, T, Tp, group,
                           hkv, q_stride, kv_stride, out_stride, window, scale, sa, n_xb);
    return hipGetLastError();
}

}  // namespace

hipError_t launch_attention_bf16(const uint16_t* q, const uint16_t* k, const uint16_t* v,
                                 void* out, int64_t batch, int64_t seq_len, int q_heads,
                                 int kv_heads, int head_dim, int64_t q_stride, int64_t kv_stride,
                                 int64_t out_stride, int64_t window, int out_mode, uint16_t* vt,
                                 hipStream_t stream) {
    // A window of seq_len or more admits every causal key.
    if (window >= seq_len) window = 0;
    const SegArgs none{0, nullptr, nullptr, nullptr};
    switch (head_dim) {
        case 64:
            return launch_attn_hd<64, 0>(q, k, v, out, batch, seq_len, q_heads, kv_heads, q_stride,
                                         kv_stride, out_stride, window, none, out_mode, vt,
                                         stream);
        case 128:
            return launch_attn_hd<128, 0>(q, k, v, out, batch, seq_len, q_heads, kv_heads,
                                          q_stride, kv_stride, out_stride, window, none, out_mode,
                                          vt, stream);
        default:
            return hipErrorInvalidValue;
    }
}

hipError_t launch_attention_bf16_seg(const uint16_t* q, const uint16_t* k, const uint16_t* v,
                                     void* out, int64_t batch, int64_t seq_len, int q_heads,
                                     int kv_heads, int head_dim, int64_t q_stride,
                                     int64_t kv_stride, int64_t out_stride, int64_t prefix,
                                     const int32_t* seg_lo, const int32_t* seg_hi,
                                     const uint64_t* pad, int out_mode, uint16_t* vt,
                                     hipStream_t stream) {
    const SegArgs sa{prefix, seg_lo, seg_hi, pad};
    switch (head_dim) {
        case 64:
            return launch_attn_hd<64, 1>(q, k, v, out, batch, seq_len, q_heads, kv_heads, q_stride,
                                         kv_stride, out_stride, 0, sa, out_mode, vt, stream);
        case 128:
            return launch_attn_hd<128, 1>(q, k, v, out, batch, seq_len, q_heads, kv_heads,
                                          q_stride, kv_stride, out_stride, 0, sa, out_mode, vt,
                                          stream);
        default:
            return hipErrorInvalidValue;
    }
}

}  // namespace ncm
