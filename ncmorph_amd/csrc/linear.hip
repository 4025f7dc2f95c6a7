// bf16-weight linear y = x * W^T on gfx950 bf16 MFMA, fp32 accumulation.
// Device counterpart of matmul_bf16_impl (packages/kernels/root.zig:106-142)
// and of the f32 widen that feeds it at load time (packages/bf16/root.zig:31-37
// via src/loader.zig:339-342): the MFMA consumes the bf16 bits directly.
#include "gemm_core.h"
#include "linear.h"

namespace ncm {

template <class S, int OUT_MODE, bool HAS_BIAS>
__global__ __launch_bounds__(S::NT, 1) void linear_kernel(const uint16_t* __restrict__ x,
                                                          const uint16_t* __restrict__ w,
                                                          const uint16_t* __restrict__ bias,
                                                          void* __restrict__ y, int64_t M,
                                                          int64_t K, int64_t N, int tiles_n,
                                                          int group_m) {
    extern __shared__ __attribute__((aligned(16))) char lds[];

    // XCD-aware grouped tile order: a run of consecutive logical ids covers a
    // group_m x tiles_n band, and each XCD receives one contiguous run.
    const int logical = xcd_remap((int)blockIdx.x, (int)gridDim.x);
    const int per_group = group_m * tiles_n;
    const int g = logical / per_group;
    const int tiles_m = (int)((M + S::BM - 1) / S::BM);
    const int gm = min(group_m, tiles_m - g * group_m);
    const int in_g = logical % per_group;
    const int tm = g * group_m + in_g % gm;
    const int tn = in_g / gm;

    const int64_t m0 = (int64_t)tm * S::BM;
    const int64_t n0 = (int64_t)tn * S::BN;

    GemmAcc<S> acc;
    acc.zero();
    gemm_mainloop<S>(x + m0 * K, K, operand_bytes(M, m0, K), w + n0 * K, K,
                     operand_bytes(N, n0, K), K, lds, acc);

    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int wm = wave % S::WGM;
    const int wn = wave / S::WGM;
#pragma unroll
    for (int nb = 0; nb < S::NB; ++nb) {
        const int64_t n = n0 + wn * S::WN + nb * 32 + (lane & 31);
        if (n >= N) continue;
        float bv = 0.0f;
        if (HAS_BIAS) bv = __uint_as_float((uint32_t)bias[n] << 16);
#pragma unroll
        for (int mb = 0; mb < S::MB; ++mb) {
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const int64_t m =
                    m0 + wm * S::WM + mb * 32 + 8 * (i >> 2) + 4 * (lane >> 5) + (i & 3);
                if (m >= M) continue;
                float v = acc.v[mb][nb][i];
                if (HAS_BIAS) v = v + bv;
                if (OUT_MODE == NCM_OUT_F32) {
                    ((float*)y)[m * N + n] = v;
                } else {
                    const uint32_t bits = bf16_bits_rne(flush_subnormal(v));
                    if (OUT_MODE == NCM_OUT_BF16_F32)
                        ((float*)y)[m * N + n] = __uint_as_float(bits << 16);
                    else
                        ((uint16_t*)y)[m * N + n] = (uint16_t)bits;
                }
            }
        }
    }
}

template <class S, int OUT_MODE, bool HAS_BIAS>
static hipError_t launch_linear_t(const uint16_t* x, const uint16_t* w, const uint16_t* bias,
                                  void* y, int64_t M, int64_t K, int64_t N,
                                  hipStream_t stream) {
    auto kern = linear_kernel<S, OUT_MODE, HAS_BIAS>;
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
    hipLaunchKernelGGL(kern, dim3(tiles_m * tiles_n), dim3(S::NT), S::LDS_BYTES, stream, x, w,
                       bias, y, M, K, N, tiles_n, group_m);
    return hipGetLastError();
}

template <class S>
static hipError_t launch_linear_s(const uint16_t* x, const uint16_t* w, const uint16_t* bias,
                                  void* y, int64_t M, int64_t K, int64_t N, int out_mode,
                                  hipStream_t st) {
    const bool hb = bias != nullptr;
    switch (out_mode) {
        case NCM_OUT_F32:
            return hb ? launch_linear_t<S, NCM_OUT_F32, true>(x, w, bias, y, M, K, N, st)
                      : launch_linear_t<S, NCM_OUT_F32, false>(x, w, bias, y, M, K, N, st);
        case NCM_OUT_BF16_F32:
            return hb ? launch_linear_t<S, NCM_OUT_BF16_F32, true>(x, w, bias, y, M, K, N, st)
                      : launch_linear_t<S, NCM_OUT_BF16_F32, false>(x, w, bias, y, M, K, N, st);
        default:
            return hb ? launch_linear_t<S, NCM_OUT_BF16, true>(x, w, bias, y, M, K, N, st)
                      : launch_linear_t<S, NCM_OUT_BF16, false>(x, w, bias, y, M, K, N, st);
    }
}

using LinBig = GemmShape<256, 256, 64, 2, 2>;
using LinMid = GemmShape<256, 128, 64, 2, 2>;
using LinSmall = GemmShape<128, 128, 64, 2, 2>;

int linear_tile_config(int64_t M, int64_t N, int forced) {
    if (forced >= 0 && forced <= 2) return forced;
    const int64_t cus = 256;
    auto tiles = [&](int64_t bm, int64_t bn) { return ((M + bm - 1) / bm) * ((N + bn - 1) / bn); };
    if (tiles(256, 256) >= cus) return 0;
    if (tiles(256, 128) >= cus) return 1;
    return 2;
}

hipError_t launch_linear(const uint16_t* x, const uint16_t* w, const uint16_t* bias, void* y,
                         int64_t M, int64_t K, int64_t N, int out_mode, int config,
                         hipStream_t stream) {
    switch (linear_tile_config(M, N, config)) {
        case 0: return launch_linear_s<LinBig>(x, w, bias, y, M, K, N, out_mode, stream);
        case 1: return launch_linear_s<LinMid>(x, w, bias, y, M, K, N, out_mode, stream);
        default: return launch_linear_s<LinSmall>(x, w, bias, y, M, K, N, out_mode, stream);
    }
}

}  // namespace ncm
