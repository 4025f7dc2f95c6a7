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
// scale = expf(log_inv_T) / d_scale computed once per call and d_scale the
// f64 sum of E_sq rounded to fp32 after the division by V.
#include "gemm_core.h"
#include "linear.h"

namespace ncm {

// scale[0] = expf(log_inv_T) / (float)(sum_k csq[k] / v), one block.
__global__ __launch_bounds__(256) void tied_head_scale_kernel(const float* __restrict__ csq,
                                                              int64_t v, float log_inv_t,
                                                              float* __restrict__ scale) {
    double s = 0.0;
    for (int64_t k = threadIdx.x; k < v; k += 256) s += (double)csq[k];
    __shared__ double red[256];
    red[threadIdx.x] = s;
    __syncthreads();
    for (int w = 128; w > 0; w >>= 1) {
        if ((int)threadIdx.x < w) red[threadIdx.x] += red[threadIdx.x + w];
        __syncthreads();
    }
    if (threadIdx.x == 0) {
        const float d_scale = (float)(red[0] / (double)v);
        scale[0] = expf(log_inv_t) / d_scale;
    }
}

template <class S, bool HAS_BIAS>
__global__ __launch_bounds__(S::NT)
__attribute__((amdgpu_waves_per_eu(S::OCC, S::OCC))) void tied_head_kernel(
    const uint16_t* __restrict__ z, const uint16_t* __restrict__ cb, const float* __restrict__ csq,
    const float* __restrict__ bias, const float* __restrict__ scale_p, float* __restrict__ y,
    int64_t M, int64_t K, int64_t N, int tiles_n, int group_m) {
    extern __shared__ __attribute__((aligned(16))) char lds[];
    // XCD-aware grouped tile order, as in the linear.
    const int logical = xcd_remap((int)blockIdx.x, (int)gridDim.x);
    const int per_group = group_m * tiles_n;
    const int g = logical / per_group;
    const int tiles_m = (int)((M + S::BM - 1) / S::BM);
    const int gm = min(group_m, tiles_m - g * group_m);
    const int in_g = logical % per_group;
    const int64_t m0 = (int64_t)(g * group_m + in_g % gm) * S::BM;
    const int64_t n0 = (int64_t)(in_g / gm) * S::BN;

    GemmAcc<S> acc;
    acc.zero();
    gemm_mainloop<S>(z + m0 * K, K, operand_bytes(M, m0, K), cb + n0 * K, K,
                     operand_bytes(N, n0, K), K, lds, acc);

    const float scale = scale_p[0];
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

template <class S, bool HAS_BIAS>
static hipError_t launch_head_t(const uint16_t* z, const uint16_t* cb, const float* csq,
                                const float* bias, const float* scale, float* y, int64_t M,
                                int64_t K, int64_t N, hipStream_t st) {
    auto kern = tied_head_kernel<S, HAS_BIAS>;
    static bool attr_set = false;
    if (!attr_set) {
        hipError_t e = hipFuncSetAttribute((const void*)kern,
                                           hipFuncAttributeMaxDynamicSharedMemorySize,
                                           S::LDS_BYTES);
        if (e != hipSuccess) return e;
        attr_set = true;
    }
    const int tiles_m = (int)((M + S::BM - 1) / S::BM);
    const int tiles_n = (int)((N + S::BN - 1) / S::BN);
    const int group_m = tiles_m < 4 ? tiles_m : 4;
    hipLaunchKernelGGL(kern, dim3(tiles_m * tiles_n), dim3(S::NT), S::LDS_BYTES, st, z, cb, csq,
                       bias, scale, y, M, K, N, tiles_n, group_m);
    return hipGetLastError();
}

hipError_t launch_tied_head(const uint16_t* z, const uint16_t* cb, const float* csq,
                            const float* bias, float log_inv_t, float* scale, float* y,
                            int64_t M, int64_t K, int64_t N, hipStream_t st) {
    hipLaunchKernelGGL(tied_head_scale_kernel, dim3(1), dim3(256), 0, st, csq, N, log_inv_t,
                       scale);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    // The linear's tile shapes and automatic choice.
    using H0 = GemmShape<256, 256, 64, 4, 2, 2, 8, true, 2, false, 1, -1, 2>;
    using H1 = GemmShape<128, 128, 64, 2, 2, 2, 8, true, 4>;
    using H2 = GemmShape<128, 128, 64, 2, 2, 2, 4, true>;
    using H5 = GemmShape<256, 128, 64, 4, 2, 2, 8, true, 3>;
    const bool hb = bias != nullptr;
#define NCM_HEAD(SH) \
    (hb ? launch_head_t<SH, true>(z, cb, csq, bias, scale, y, M, K, N, st) \
        : launch_head_t<SH, false>(z, cb, csq, bias, scale, y, M, K, N, st))
    switch (linear_tile_config(M, N, K, -1)) {
        case 0: return NCM_HEAD(H0);
        case 1: return NCM_HEAD(H1);
        case 5: return NCM_HEAD(H5);
        default: return NCM_HEAD(H2);
    }
#undef NCM_HEAD
}

}  // namespace ncm
