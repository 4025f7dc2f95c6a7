// Linear y = x * W^T on gfx950 MFMA, fp32 accumulation.
// bf16 operands: device counterpart of matmul_bf16_impl
// (packages/kernels/root.zig:106-142) and of the f32 widen that feeds it at
// load time (packages/bf16/root.zig:31-37 via src/loader.zig:339-342): the
// MFMA consumes the bf16 bits directly.
// fp32 operands: device counterpart of matmul (packages/kernels/root.zig:25-65)
// on the fp32 MFMA.
#include <cstdlib>

#include "gemm_core.h"
#include "linear.h"

namespace ncm {

// HAS_RES: y = residual + result (the decoder's add_rows, src/decoder.zig:279-282):
// fp32 output adds in fp32; the bf16 modes round the linear's result to bf16
// first (its own output contract) and then round the sum to bf16. residual
// [M, N] fp32 may be y itself (each element is read, then written, by one
// thread).
template <class S, int OUT_MODE, bool HAS_BIAS, bool HAS_RES = false>
__global__ __launch_bounds__(S::NT)
__attribute__((amdgpu_waves_per_eu(S::OCC, S::OCC))) void linear_kernel(const void* __restrict__ x,
                                                          const void* __restrict__ w,
                                                          const uint16_t* __restrict__ bias,
                                                          void* y, int64_t M,
                                                          int64_t K, int64_t N, int tiles_n,
                                                          int group_m, const float* residual) {
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
    gemm_mainloop<S>((const char*)x + m0 * K * S::ESZ, K, operand_bytes(M, m0, K, S::ESZ),
                     (const char*)w + n0 * K * S::ESZ, K, operand_bytes(N, n0, K, S::ESZ), K, lds,
                     acc);

    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    if (wave >= S::NWG) return;  // K group 1: its sums were handed to group 0
    const int wm = wave % S::WGM;
    const int wn = wave / S::WGM;
    if (m0 + S::BM <= M && n0 + S::BN <= N && (N & 3) == 0 && ((uintptr_t)y & 15) == 0 &&
        (!HAS_RES || ((uintptr_t)residual & 15) == 0)) {
        // Whole tile in range: transpose each 4-row group of the D fragment
        // inside lane quads so that every lane stores 4 consecutive columns
        // of one row (16-byte stores; 8 lanes cover 128 contiguous bytes).
        // The output is not read again by this kernel: non-temporal stores.
        const int q = lane & 3;
        const int col4 = (lane & 31) & ~3;
        const int hrow = 4 * (lane >> 5) + q;
#pragma unroll
        for (int nb = 0; nb < S::NB; ++nb) {
            float bv = 0.0f;
            if (HAS_BIAS) bv = __uint_as_float((uint32_t)bias[n0 + wn * S::WN + nb * 32 + (lane & 31)] << 16);
            const int64_t ncol = n0 + wn * S::WN + nb * 32 + col4;
#pragma unroll
            for (int mb = 0; mb < S::MB; ++mb) {
#pragma unroll
                for (int blk = 0; blk < 4; ++blk) {
                    float v[4];
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        v[j] = acc.v[mb][nb][4 * blk + j];
                        if (HAS_BIAS) v[j] = v[j] + bv;
                    }
                    quad_transpose4(v, q);
                    const int64_t m = m0 + wm * S::WM + mb * 32 + 8 * blk + hrow;
                    f32x4_t rv;
                    if (HAS_RES) rv = *(const f32x4_t*)(residual + m * N + ncol);
                    if (OUT_MODE == NCM_OUT_F32) {
                        f32x4_t o;
                        o[0] = v[0]; o[1] = v[1]; o[2] = v[2]; o[3] = v[3];
                        if (HAS_RES)
#pragma unroll
                            for (int j = 0; j < 4; ++j) o[j] = rv[j] + o[j];
                        __builtin_nontemporal_store(o, (f32x4_t*)((float*)y + m * N + ncol));
                    } else {
                        // bf16(flush(v)) (then bf16(residual + that)) for two
                        // columns per v_cvt_pk_bf16_f32; the NaN rule on the
                        // stored rounding only (a NaN stays a NaN through the
                        // residual add).
                        uint32_t pr[2];
#pragma unroll
                        for (int h = 0; h < 2; ++h) {
                            const float f0 = flush_subnormal(v[2 * h]);
                            const float f1 = flush_subnormal(v[2 * h + 1]);
                            if (HAS_RES) {
                                const uint32_t t = bf16x2_rne(f0, f1);
                                pr[h] = bf16x2_bits_rne(rv[2 * h] + __uint_as_float(t << 16),
                                                        rv[2 * h + 1] +
                                                            __uint_as_float(t & 0xFFFF0000u));
                            } else {
                                pr[h] = bf16x2_bits_rne(f0, f1);
                            }
                        }
                        if (OUT_MODE == NCM_OUT_BF16_F32) {
                            u32x4_t o;
                            o[0] = pr[0] << 16; o[1] = pr[0] & 0xFFFF0000u;
                            o[2] = pr[1] << 16; o[3] = pr[1] & 0xFFFF0000u;
                            __builtin_nontemporal_store(o, (u32x4_t*)((float*)y + m * N + ncol));
                        } else {
                            u32x2_t o;
                            o[0] = pr[0];
                            o[1] = pr[1];
                            __builtin_nontemporal_store(o, (u32x2_t*)((uint16_t*)y + m * N + ncol));
                        }
                    }
                }
            }
        }
        return;
    }
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
                    ((float*)y)[m * N + n] = HAS_RES ? residual[m * N + n] + v : v;
                } else {
                    uint32_t bits = bf16_bits_rne(flush_subnormal(v));
                    if (HAS_RES) bits = bf16_bits_rne(residual[m * N + n] + __uint_as_float(bits << 16));
                    if (OUT_MODE == NCM_OUT_BF16_F32)
                        ((float*)y)[m * N + n] = __uint_as_float(bits << 16);
                    else
                        ((uint16_t*)y)[m * N + n] = (uint16_t)bits;
                }
            }
        }
    }
}

template <class S, int OUT_MODE, bool HAS_BIAS, bool HAS_RES = false>
static hipError_t launch_linear_t(const void* x, const void* w, const uint16_t* bias, void* y,
                                  int64_t M, int64_t K, int64_t N, hipStream_t stream,
                                  const float* residual = nullptr) {
    auto kern = linear_kernel<S, OUT_MODE, HAS_BIAS, HAS_RES>;
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
                       bias, y, M, K, N, tiles_n, group_m, residual);
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

// Tile configurations of the bf16 linear (index = NCM_LINEAR_TILE):
//  0: 256x256x64, 8 waves (64x128 each, 2 per SIMD), direct-to-LDS loads,
//     2 LDS stages; SCHED 8: loads and fragment reads interleaved between
//     the MFMAs of the first two k-steps, barrier in the middle of the last
//     k-step
//  1: 128x128x64, 8 waves (32x64, 2 per SIMD), DMA, SCHED 8, 4 LDS stages,
//     16x16x32 MFMAs
//  2: 128x128x64, 4 waves, DMA, fences (SCHED 4), 2 stages: two workgroups
//     per CU
//  3: 256x256x32, 8 waves, DMA, ping-pong (SCHED 6), 4 LDS stages
//  4: 256x256x64, 4 waves (128x128, 1 per SIMD), DMA, SCHED 5
//  5: 256x128x64, 8 waves (64x64), DMA, SCHED 8, 3 LDS stages
//  6: 256x256x64, 8 waves, register-staged loads, fences
//  7: 128x128x64, 4 waves, register-staged loads, fences
//  8: 128x128x32, two K groups of 4 waves (SCHED 7: 8 waves, two per SIMD,
//     alternate K tiles from 8 LDS stages, summed through LDS at the end)
//  9: as 8 with 128x128x64 tiles and 4 LDS stages
// 10: 128x128x128 (256-byte rows), 4 waves, DMA, SCHED 5, 2 stages
// 11, 12, 13: as 0, 1 and 5 with SCHED 5 (all loads of a tile issued
//     together at its start, fragment reads of a k-step as one group)
using Lin0 = GemmShape<256, 256, 64, 4, 2, 2, 8, true, 2, false, 1, -1, -1, true>;
using Lin1 = GemmShape<128, 128, 64, 4, 2, 2, 8, true, 4, false, 1, -1, -1, true>;
using Lin2 = GemmShape<128, 128, 64, 2, 2, 2, 4, true>;
using Lin3 = GemmShape<256, 256, 32, 4, 2, 2, 6, true, 4>;
using Lin4 = GemmShape<256, 256, 64, 2, 2, 1, 5, true>;
using Lin5 = GemmShape<256, 128, 64, 4, 2, 2, 8, true, 3, false, 1, -1, -1, true>;
using Lin6 = GemmShape<256, 256, 64, 4, 2, 2, 4, false>;
using Lin7 = GemmShape<128, 128, 64, 2, 2, 2, 4, false>;
using Lin8 = GemmShape<128, 128, 32, 2, 2, 2, 7, true, 8, false, 2>;
using Lin9 = GemmShape<128, 128, 64, 2, 2, 2, 7, true, 4, false, 2>;
using Lin10 = GemmShape<128, 128, 128, 2, 2, 2, 5, true, 2>;
using Lin11 = GemmShape<256, 256, 64, 4, 2, 2, 5, true>;
using Lin12 = GemmShape<128, 128, 64, 2, 2, 2, 5, true, 4>;
using Lin13 = GemmShape<256, 128, 64, 4, 2, 2, 5, true, 3>;
using Lin14 = GemmShape<256, 256, 64, 4, 2, 2, 8, true, 2, false, 1, -1, 2>;
using Lin15 = GemmShape<256, 128, 64, 4, 2, 2, 8, true, 3>;
constexpr int kLinConfigs = 16;

// fp32 linear: 128x128x32 (128-byte rows), 4 waves, DMA, SCHED 5, two
// stages (64 KB: two workgroups per CU). The fp32 MFMA has 1/16 of the bf16
// rate, so this tile is MFMA-bound with a wide margin.
using LinF32 = GemmShape<128, 128, 32, 2, 2, 2, 5, true, 2, true>;

int linear_tile_config(int64_t M, int64_t N, int64_t K, int forced) {
    if (forced >= 0 && forced < kLinConfigs) return forced;
    const int64_t cus = 256;
    auto tiles = [&](int64_t bm, int64_t bn) { return ((M + bm - 1) / bm) * ((N + bn - 1) / bn); };
    // 256x256 with 8 waves when it fills at least three quarters of the
    // CUs; 128x128 with four LDS stages when that gives at most one tile per
    // CU (latency-bound: deeper prefetch pays); 256x128 with three stages
    // when its tiles fill the CUs about once or twice; else 128x128 with two
    // stages (two workgroups per CU). All with direct-to-LDS loads.
    // (Measured on the decoder's and the benchmark's shapes.)
    if (tiles(256, 256) * 4 >= cus * 3) return 0;
    if (tiles(128, 128) <= cus) return 1;
    if (tiles(256, 128) * 4 >= cus * 3 && tiles(256, 128) <= 2 * cus) return 5;
    return 2;
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
    if (config < 0) {
        // A partial last row tile that would add a round: its rows go to the
        // tail kernel.
        const int64_t r = linear_tail_rows(M, N, K);
        if (r > 0) {
            const int64_t mm = M - r;
            hipError_t e = launch_linear(x, w, bias, y, mm, K, N, out_mode, 0, stream);
            if (e != hipSuccess) return e;
            const size_t esz = out_mode == NCM_OUT_BF16 ? 2 : 4;
            return launch_linear_tail(x + mm * K, w, bias, nullptr, (char*)y + mm * N * esz, r,
                                      K, N, out_mode, false, stream);
        }
    }
    switch (linear_tile_config(M, N, K, config)) {
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
        default: return launch_linear_s<Lin15>(x, w, bias, y, M, K, N, out_mode, stream);
    }
}

template <class S>
static hipError_t launch_linear_res_s(const uint16_t* x, const uint16_t* w, const uint16_t* bias,
                                      const float* res, void* y, int64_t M, int64_t K, int64_t N,
                                      int out_mode, hipStream_t st) {
    const bool hb = bias != nullptr;
#define NCM_LINR(MODE, HB) launch_linear_t<S, MODE, HB, true>(x, w, bias, y, M, K, N, st, res)
    switch (out_mode) {
        case NCM_OUT_F32: return hb ? NCM_LINR(NCM_OUT_F32, true) : NCM_LINR(NCM_OUT_F32, false);
        case NCM_OUT_BF16_F32:
            return hb ? NCM_LINR(NCM_OUT_BF16_F32, true) : NCM_LINR(NCM_OUT_BF16_F32, false);
        default: return hb ? NCM_LINR(NCM_OUT_BF16, true) : NCM_LINR(NCM_OUT_BF16, false);
    }
#undef NCM_LINR
}

hipError_t launch_linear_residual(const uint16_t* x, const uint16_t* w, const uint16_t* bias,
                                  const float* residual, void* y, int64_t M, int64_t K,
                                  int64_t N, int out_mode, hipStream_t stream) {
    // The automatic tile choice only (configurations 0, 1, 2 and 5), with
    // the tail rows of linear_tail_rows on the tail kernel.
    const int64_t r = linear_tail_rows(M, N, K);
    if (r > 0) {
        const int64_t mm = M - r;
        hipError_t e =
            launch_linear_residual(x, w, bias, residual, y, mm, K, N, out_mode, stream);
        if (e != hipSuccess) return e;
        const size_t esz = out_mode == NCM_OUT_BF16 ? 2 : 4;
        return launch_linear_tail(x + mm * K, w, bias, residual + mm * N,
                                  (char*)y + mm * N * esz, r, K, N, out_mode, false, stream);
    }
    switch (linear_tile_config(M, N, K, -1)) {
        case 0: return launch_linear_res_s<Lin0>(x, w, bias, residual, y, M, K, N, out_mode, stream);
        case 1: return launch_linear_res_s<Lin1>(x, w, bias, residual, y, M, K, N, out_mode, stream);
        case 5: return launch_linear_res_s<Lin5>(x, w, bias, residual, y, M, K, N, out_mode, stream);
        default: return launch_linear_res_s<Lin2>(x, w, bias, residual, y, M, K, N, out_mode, stream);
    }
}

hipError_t launch_linear_f32(const float* x, const float* w, float* y, int64_t M, int64_t K,
                             int64_t N, hipStream_t stream) {
    return launch_linear_t<LinF32, NCM_OUT_F32, false>(x, w, nullptr, y, M, K, N, stream);
}

}  // namespace ncm
