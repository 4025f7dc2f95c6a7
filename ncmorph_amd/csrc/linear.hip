// bf16-weight linear y = x * W^T on gfx950 bf16 MFMA, fp32 accumulation.
// Device counterpart of matmul_bf16_impl (packages/kernels/root.zig:106-142)
// and of the f32 widen that feeds it at load time (packages/bf16/root.zig:31-37
// via src/loader.zig:339-342): the MFMA consumes the bf16 bits directly.
#include <cstdlib>

#include "gemm_core.h"
#include "linear.h"

namespace ncm {

template <class S, int OUT_MODE, bool HAS_BIAS>
__global__ __launch_bounds__(S::NT)
__attribute__((amdgpu_waves_per_eu(S::OCC, S::OCC))) void linear_kernel(const uint16_t* __restrict__ x,
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

// Tile configurations (index = NCM_LINEAR_TILE):
//  0: 256x256x64, 4 waves (128x128 each), 1 wave/SIMD
//  1: 256x128x32, 4 waves (128x64), 2 waves/SIMD
//  2: 128x128x64, 4 waves (64x64), 2 waves/SIMD
//  3: 128x128x64, fragment double buffering, 2 waves/SIMD
//  4: 256x128x64, 4 waves (128x64), 1 wave/SIMD, two prefetch sets
//  5: 128x64x64, 4 waves (64x32), 2 waves/SIMD
//  6: 256x256x64, two prefetch sets
//  7: 256x256x64, fragment double buffering
//  8: 256x256x32, two prefetch sets, fragment double buffering
//  9: 256x256x64, fragment double buffering, explicit DS/MFMA interleave
// 10: 256x256x64, iglp_opt(0)
// 11: 256x256x64, iglp_opt(1)
// 12: 256x256x64, two prefetch sets, FDB, explicit interleave
// 13: 256x256x64, FDB, scheduling fences
// 14: 256x256x64, two prefetch sets, FDB, scheduling fences
// 15: 256x128x64, FDB, scheduling fences, 1 wave/SIMD
// 16: 256x256x64, 8 waves (128x64 each, 2 per SIMD), FDB, fences
// 17: 256x256x64, 8 waves, FDB, compiler order
// 18: 256x256x32, 8 waves, FDB, fences
// 19: 256x256x64, 8 waves (64x128 each), FDB, fences
// 20: 256x128x32, 2 waves/SIMD (two workgroups per CU), FDB, fences
// 21: 128x128x64, 2 waves/SIMD, FDB, fences
// 22: 256x128x32, 2 waves/SIMD, two prefetch sets, FDB, fences
// 23: 128x256x32, 2 waves/SIMD, FDB, fences
// 24: 256x256x64, direct-to-LDS loads, FDB, fences
// 25: 256x256x64, 8 waves (64x128), direct-to-LDS loads, FDB, fences
// 26: 128x128x64, direct-to-LDS loads, FDB, fences, 2 waves/SIMD
// 27: 256x128x64, direct-to-LDS loads, FDB, fences
using Lin0 = GemmShape<256, 256, 64, 2, 2, 1, 1, false>;
using Lin1 = GemmShape<256, 128, 32, 2, 2, 1, 2, false>;
using Lin2 = GemmShape<128, 128, 64, 2, 2, 1, 2, false>;
using Lin3 = GemmShape<128, 128, 64, 2, 2, 1, 2, true>;
using Lin4 = GemmShape<256, 128, 64, 2, 2, 2, 1, true>;
using Lin5 = GemmShape<128, 64, 64, 2, 2, 1, 2, false>;
using Lin6 = GemmShape<256, 256, 64, 2, 2, 2, 1, false>;
using Lin7 = GemmShape<256, 256, 64, 2, 2, 1, 1, true>;
using Lin8 = GemmShape<256, 256, 32, 2, 2, 2, 1, true>;
using Lin9 = GemmShape<256, 256, 64, 2, 2, 1, 1, true, 3>;
using Lin10 = GemmShape<256, 256, 64, 2, 2, 1, 1, false, 1>;
using Lin11 = GemmShape<256, 256, 64, 2, 2, 1, 1, false, 2>;
using Lin12 = GemmShape<256, 256, 64, 2, 2, 2, 1, true, 3>;
using Lin13 = GemmShape<256, 256, 64, 2, 2, 1, 1, true, 4>;
using Lin14 = GemmShape<256, 256, 64, 2, 2, 2, 1, true, 4>;
using Lin15 = GemmShape<256, 128, 64, 2, 2, 1, 1, true, 4>;
using Lin16 = GemmShape<256, 256, 64, 2, 4, 1, 2, true, 4>;
using Lin17 = GemmShape<256, 256, 64, 2, 4, 1, 2, true, 0>;
using Lin18 = GemmShape<256, 256, 32, 2, 4, 1, 2, true, 4>;
using Lin19 = GemmShape<256, 256, 64, 4, 2, 1, 2, true, 4>;
using Lin20 = GemmShape<256, 128, 32, 2, 2, 1, 2, true, 4>;
using Lin21 = GemmShape<128, 128, 64, 2, 2, 1, 2, true, 4>;
using Lin22 = GemmShape<256, 128, 32, 2, 2, 2, 2, true, 4>;
using Lin23 = GemmShape<128, 256, 32, 2, 2, 1, 2, true, 4>;
using Lin24 = GemmShape<256, 256, 64, 2, 2, 1, 1, true, 4, true>;
using Lin25 = GemmShape<256, 256, 64, 4, 2, 1, 2, true, 4, true>;
using Lin26 = GemmShape<128, 128, 64, 2, 2, 1, 2, true, 4, true>;
using Lin27 = GemmShape<256, 128, 64, 2, 2, 1, 1, true, 4, true>;
constexpr int kLinConfigs = 28;

int linear_tile_config(int64_t M, int64_t N, int forced) {
    if (forced >= 0 && forced < kLinConfigs) return forced;
    const int64_t cus = 256;
    auto tiles = [&](int64_t bm, int64_t bn) { return ((M + bm - 1) / bm) * ((N + bn - 1) / bn); };
    // 256x256 with 8 waves when it fills every CU, else 128x128 (two
    // workgroups per CU); both with direct-to-LDS loads.
    if (tiles(256, 256) >= cus) return 25;
    return 26;
}

hipError_t launch_linear(const uint16_t* x, const uint16_t* w, const uint16_t* bias, void* y,
                         int64_t M, int64_t K, int64_t N, int out_mode, int config,
                         hipStream_t stream) {
    // NCM_LINEAR_TILE pins the tile configuration (tuning sweeps).
    static const int env_cfg = [] {
        const char* e = getenv("NCM_LINEAR_TILE");
        return e ? atoi(e) : -1;
    }();
    if (config < 0) config = env_cfg;
    switch (linear_tile_config(M, N, config)) {
        case 0: return launch_linear_s<Lin0>(x, w, bias, y, M, K, N, out_mode, stream);
        case 1: return launch_linear_s<Lin1>(x, w, bias, y, M, K, N, out_mode, stream);
        case 2: return launch_linear_s<Lin2>(x, w, bias, y, M, K, N, out_mode, stream);
        case 3: return launch_linear_s<Lin3>(x, w, bias, y, M, K, N, out_mode, stream);
        case 4: return launch_linear_s<Lin4>(x, w, bias, y, M, K, N, out_mode, stream);
        case 5: return launch_linear_s<Lin5>(x, w, bias, y, M, K, N, out_mode, stream);
        case 6: return launch_linear_s<Lin6>(x, w, bias, y, M, K, N, out_mode, stream);
        case 7: return launch_linear_s<Lin7>(x, w, bias, y, M, K, N, out_mode, stream);
        case 8: return launch_linear_s<Lin8>(x, w, bias, y, M, K, N, out_mode, stream);
        case 9: return launch_linear_s<Lin9>(x, w, bias, y, M, K, N, out_mode, stream);
        case 10: return launch_linear_s<Lin10>(x, w, bias, y, M, K, N, out_mode, stream);
        case 11: return launch_linear_s<Lin11>(x, w, bias, y, M, K, N, out_mode, stream);
        case 12: return launch_linear_s<Lin12>(x, w, bias, y, M, K, N, out_mode, stream);
        case 13: return launch_linear_s<Lin13>(x, w, bias, y, M, K, N, out_mode, stream);
        case 14: return launch_linear_s<Lin14>(x, w, bias, y, M, K, N, out_mode, stream);
        case 15: return launch_linear_s<Lin15>(x, w, bias, y, M, K, N, out_mode, stream);
        case 16: return launch_linear_s<Lin16>(x, w, bias, y, M, K, N, out_mode, stream);
        case 17: return launch_linear_s<Lin17>(x, w, bias, y, M, K, N, out_mode, stream);
        case 18: return launch_linear_s<Lin18>(x, w, bias, y, M, K, N, out_mode, stream);
        case 19: return launch_linear_s<Lin19>(x, w, bias, y, M, K, N, out_mode, stream);
        case 20: return launch_linear_s<Lin20>(x, w, bias, y, M, K, N, out_mode, stream);
        case 21: return launch_linear_s<Lin21>(x, w, bias, y, M, K, N, out_mode, stream);
        case 22: return launch_linear_s<Lin22>(x, w, bias, y, M, K, N, out_mode, stream);
        case 23: return launch_linear_s<Lin23>(x, w, bias, y, M, K, N, out_mode, stream);
        case 24: return launch_linear_s<Lin24>(x, w, bias, y, M, K, N, out_mode, stream);
        case 25: return launch_linear_s<Lin25>(x, w, bias, y, M, K, N, out_mode, stream);
        case 26: return launch_linear_s<Lin26>(x, w, bias, y, M, K, N, out_mode, stream);
        default: return launch_linear_s<Lin27>(x, w, bias, y, M, K, N, out_mode, stream);
    }
}

}  // namespace ncm
