// Codebook-tied code head of the NCM generator on gfx950 MFMA.
//
// The reference describes the head (PROJECT.md:222, upstream
// _TiedCodebookHead) and has no code for it yet: with the level's codebook
// E [V, d] and E_sq[k] = ||E_k||^2,
//   d_scale = mean_k E_sq[k]
//   logits[r, k] = (2 z_r . E_k - E_sq[k]) / d_scale * exp(log_inv_T) (+ bias[k])
// It is the RVQ distance with the sign flipped and a per-level scale: the same
// bf16 MFMA main loop (z rows against codebook rows, fp32 accumulate) with
// E_sq from ncm_rvq_prepare, and the affine map fused into the epilogue.
// fp32 operation order of the epilogue (tolerance-based parity, like the
// linear): t = 2 S - E_sq[k]; logit = t * scale (+ bias[k]), with
// scale = expf(log_inv_T) / d_scale computed once per level and call and
// d_scale the f64 sum of E_sq rounded to fp32 after the division by V. The
// level-parallel step evaluates every level's head at once (each level's
// positions against its own codebook), so one launch covers all levels.
#include "gemm_core.h"
#include "linear.h"

namespace ncm {

constexpr int kHeadMaxLevels = 32;

// One launch covers every level: level l owns rows [row0[l], row0[l] +
// rows[l]) of z and of the logits, codebook l, E_sq row l, bias row l and
// output tiles [tile0[l], tile0[l + 1]).
struct HeadArgs {
    const uint16_t* z;
    const uint16_t* cb;    // [levels, v, d]
    const float* csq;      // [levels, v]
    const float* bias;     // [levels, v] or null
    const float* scale;    // [levels], device
    float* y;              // [sum rows, v]
    int64_t v, d;
    int levels;
    int tiles_n;
    int64_t row0[kHeadMaxLevels];
    int64_t rows[kHeadMaxLevels];
    int tile0[kHeadMaxLevels + 1];
    float log_inv_t[kHeadMaxLevels];
};

// scale[l] = expf(log_inv_t[l]) / (float)(sum_k csq[l, k] / v), one block
// per level.
__global__ __launch_bounds__(256) void tied_head_scale_kernel(HeadArgs a, float* scale) {
    const int l = blockIdx.x;
    const float* c = a.csq + (int64_t)l * a.v;
    double s = 0.0;
    for (int64_t k = threadIdx.x; k < a.v; k += 256) s += (double)c[k];
    __shared__ double red[256];
    red[threadIdx.x] = s;
    __syncthreads();
    for (int w = 128; w > 0; w >>= 1) {
        if ((int)threadIdx.x < w) red[threadIdx.x] += red[threadIdx.x + w];
        __syncthreads();
    }
    if (threadIdx.x == 0) {
        const float d_scale = (float)(red[0] / (double)a.v);
        scale[l] = expf(a.log_inv_t[l]) / d_scale;
    }
}

template <class S, bool HAS_BIAS>
__global__ __launch_bounds__(S::NT)
__attribute__((amdgpu_waves_per_eu(S::OCC, S::OCC))) void tied_head_kernel(HeadArgs a) {
    extern __shared__ __attribute__((aligned(16))) char lds[];
    const int logical = xcd_remap((int)blockIdx.x, (int)gridDim.x);
    int l = 0;
    while (l + 1 < a.levels && logical >= a.tile0[l + 1]) ++l;
    // Inside the level: grouped tile order (bands of up to 4 row tiles).
    const int64_t M = a.rows[l], N = a.v, K = a.d;
    const int local = logical - a.tile0[l];
    const int tiles_m = (int)((M + S::BM - 1) / S::BM);
    const int group_m = tiles_m < 4 ? tiles_m : 4;
    const int per_group = group_m * a.tiles_n;
    const int g = local / per_group;
    const int gm = min(group_m, tiles_m - g * group_m);
    const int in_g = local % per_group;
    const int64_t m0 = (int64_t)(g * group_m + in_g % gm) * S::BM;
    const int64_t n0 = (int64_t)(in_g / gm) * S::BN;
    const uint16_t* z = a.z + a.row0[l] * K;
    const uint16_t* cb = a.cb + (int64_t)l * N * K;
    const float* csq = a.csq + (int64_t)l * N;
    const float* bias = HAS_BIAS ? a.bias + (int64_t)l * N : nullptr;
    float* y = a.y + a.row0[l] * N;

    GemmAcc<S> acc;
    acc.zero();
    gemm_mainloop<S>(z + m0 * K, K, operand_bytes(M, m0, K), cb + n0 * K, K,
                     operand_bytes(N, n0, K), K, lds, acc);

    const float scale = a.scale[l];
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int wm = wave % S::WGM;
    const int wn = wave / S::WGM;
    auto logit = [&](float s, float c, float b) {
        const float t = 2.0f * s - c;
        const float r = t * scale;
        return HAS_BIAS ? r + b : r;
    };
    if (m0 + S::BM <= M && n0 + S::BN <= N && (N & 3) == 0 && ((uintptr_t)y & 15) == 0 &&
        ((uintptr_t)csq & 15) == 0 && (!HAS_BIAS || ((uintptr_t)bias & 15) == 0)) {
        // Whole tile: after the quad transpose every lane holds 4 consecutive
        // codes of one row (16-byte loads of E_sq and bias, 16-byte stores).
        const int q = lane & 3;
        const int col4 = (lane & 31) & ~3;
        const int hrow = 4 * (lane >> 5) + q;
#pragma unroll
        for (int nb = 0; nb < S::NB; ++nb) {
            const int64_t ncol = n0 + wn * S::WN + nb * 32 + col4;
            const f32x4_t c4 = *(const f32x4_t*)(csq + ncol);
            f32x4_t b4 = {0.0f, 0.0f, 0.0f, 0.0f};
            if (HAS_BIAS) b4 = *(const f32x4_t*)(bias + ncol);
#pragma unroll
            for (int mb = 0; mb < S::MB; ++mb) {
#pragma unroll
                for (int blk = 0; blk < 4; ++blk) {
                    float v[4];
#pragma unroll
                    for (int j = 0; j < 4; ++j) v[j] = acc.v[mb][nb][4 * blk + j];
                    quad_transpose4(v, q);
                    const int64_t m = m0 + wm * S::WM + mb * 32 + 8 * blk + hrow;
                    f32x4_t o;
#pragma unroll
                    for (int j = 0; j < 4; ++j) o[j] = logit(v[j], c4[j], b4[j]);
                    __builtin_nontemporal_store(o, (f32x4_t*)(y + m * N + ncol));
                }
            }
        }
        return;
    }
#pragma unroll
    for (int nb = 0; nb < S::NB; ++nb) {
        const int64_t n = n0 + wn * S::WN + nb * 32 + (lane & 31);
        if (n >= N) continue;
        const float c = csq[n];
        const float b = HAS_BIAS ? bias[n] : 0.0f;
#pragma unroll
        for (int mb = 0; mb < S::MB; ++mb) {
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const int64_t m =
                    m0 + wm * S::WM + mb * 32 + 8 * (i >> 2) + 4 * (lane >> 5) + (i & 3);
                if (m < M) y[m * N + n] = logit(acc.v[mb][nb][i], c, b);
            }
        }
    }
}

template <class S>
static hipError_t launch_head_t(HeadArgs& a, hipStream_t st) {
    int64_t t = 0;
    const int64_t tn = (a.v + S::BN - 1) / S::BN;
    for (int l = 0; l < a.levels; ++l) {
        a.tile0[l] = (int)t;
        t += (a.rows[l] + S::BM - 1) / S::BM * tn;
        if (t > 0x7fffffff) return hipErrorInvalidConfiguration;
    }
    a.tiles_n = (int)tn;
    a.tile0[a.levels] = (int)t;
    if (t == 0) return hipSuccess;
    auto kern = a.bias ? tied_head_kernel<S, true> : tied_head_kernel<S, false>;
    static bool attr_set[2] = {false, false};
    if (!attr_set[a.bias ? 1 : 0]) {
        hipError_t e = hipFuncSetAttribute((const void*)kern,
                                           hipFuncAttributeMaxDynamicSharedMemorySize,
                                           S::LDS_BYTES);
        if (e != hipSuccess) return e;
        attr_set[a.bias ? 1 : 0] = true;
    }
    hipLaunchKernelGGL(kern, dim3((unsigned)t), dim3(S::NT), S::LDS_BYTES, st, a);
    return hipGetLastError();
}

// Levels [l0, l1) of a as a launch of their own (rows keep their places in
// y; codebooks, norms, biases and scales from level l0 on).
static HeadArgs sub_levels(const HeadArgs& a, int l0, int l1) {
    HeadArgs b = a;
    b.levels = l1 - l0;
    b.cb = a.cb + (int64_t)l0 * a.v * a.d;
    b.csq = a.csq + (int64_t)l0 * a.v;
    b.bias = a.bias ? a.bias + (int64_t)l0 * a.v : nullptr;
    b.scale = a.scale + l0;
    for (int l = 0; l < b.levels; ++l) {
        b.row0[l] = a.row0[l0 + l];
        b.rows[l] = a.rows[l0 + l];
        b.log_inv_t[l] = a.log_inv_t[l0 + l];
    }
    return b;
}

hipError_t launch_tied_head(const uint16_t* z, const uint16_t* cb, const float* csq,
                            const float* bias, const float* log_inv_t, const int64_t* rows,
                            int levels, float* scale, float* y, int64_t d, int64_t v,
                            hipStream_t st) {
    if (levels < 1 || levels > kHeadMaxLevels) return hipErrorInvalidValue;
    HeadArgs a{};
    a.z = z; a.cb = cb; a.csq = csq; a.bias = bias; a.scale = scale; a.y = y;
    a.v = v; a.d = d; a.levels = levels;
    int64_t r = 0, tiles_big = 0, tiles_small = 0;
    for (int l = 0; l < levels; ++l) {
        a.row0[l] = r;
        a.rows[l] = rows[l];
        a.log_inv_t[l] = log_inv_t[l];
        r += rows[l];
        tiles_big += ((rows[l] + 255) / 256) * ((v + 255) / 256);
        tiles_small += ((rows[l] + 127) / 128) * ((v + 127) / 128);
    }
    hipLaunchKernelGGL(tied_head_scale_kernel, dim3(levels), dim3(256), 0, st, a, scale);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    // The linear's tiles: 256 x 256 when the levels together fill three
    // quarters of the CUs with them, else 128 x 128 with four LDS stages (at
    // most about one tile per CU) or two (two workgroups per CU).
    using H0 = GemmShape<256, 256, 64, 4, 2, 2, 8, true, 2, false, 1, -1, -1, true>;
    using H1 = GemmShape<128, 128, 64, 2, 2, 2, 8, true, 4>;
    using H2 = GemmShape<128, 128, 64, 2, 2, 2, 4, true>;
    const int64_t cus = 256;
    if (tiles_big * 4 >= cus * 3) {
        // The leading levels that do not fill a 256-row tile (the NCM step's
        // 32 ... 128-position levels) go to a launch of their own on 128 x
        // 128 tiles when, without their tiles, the 256 x 256 tiles of the
        // rest need fewer rounds of the CUs: the small launch then takes a
        // fraction of a round instead of a whole one.
        int split = 0;
        int64_t rest = tiles_big, small = 0;
        while (split < levels - 1 && rows[split] < 256) {
            rest -= ((rows[split] + 255) / 256) * ((v + 255) / 256);
            small += ((rows[split] + 127) / 128) * ((v + 127) / 128);
            ++split;
        }
        if (split > 0 && small <= cus && (rest + cus - 1) / cus < (tiles_big + cus - 1) / cus) {
            HeadArgs lo = sub_levels(a, 0, split), hi = sub_levels(a, split, levels);
            hipError_t e2 = launch_head_t<H1>(lo, st);
            if (e2 != hipSuccess) return e2;
            return launch_head_t<H0>(hi, st);
        }
        return launch_head_t<H0>(a, st);
    }
    if (tiles_small <= cus) return launch_head_t<H1>(a, st);
    return launch_head_t<H2>(a, st);
}

}  // namespace ncm
