// RVQ helpers shared by the encode and decode paths: shape checks, the
// level table, the fixed-order squared codebook norms and the decode.
#include "common.h"
#include "rvq.h"

namespace ncm {

static bool pow2(int64_t s) { return s >= 1 && (s & (s - 1)) == 0; }

int rvq_check_shape(int64_t b, int64_t t, int64_t d, int64_t levels, const int32_t* strides,
                    int64_t v) {
    if (b < 1 || t < 1 || d < 64 || d % 64 != 0 || d > (int64_t(1) << 20)) return NCM_E_SHAPE;
    if (levels < 1 || levels > kMaxLevels) return NCM_E_SHAPE;
    if (v < 1 || v > 65536) return NCM_E_SHAPE;
    for (int64_t l = 0; l < levels; ++l) {
        if (!pow2(strides[l])) return NCM_E_SHAPE;
        if (l > 0 && strides[l] > strides[l - 1]) return NCM_E_SHAPE;
    }
    if (t % strides[0] != 0) return NCM_E_SHAPE;
    if (b > (int64_t(1) << 31) || t > (int64_t(1) << 31) || b * t > (int64_t(1) << 31))
        return NCM_E_SHAPE;
    return NCM_OK;
}

LevelTable make_level_table(int64_t t, int64_t levels, const int32_t* strides) {
    LevelTable L{};
    L.levels = (int32_t)levels;
    int64_t off = 0;
    for (int64_t l = 0; l < levels; ++l) {
        L.stride[l] = strides[l];
        L.offset[l] = off;
        off += t / strides[l];
    }
    L.total = off;
    return L;
}

// Fixed-order squared norm of a bf16 row (the oracle's ncmo_sumsq_bf16_fixed):
// lane j accumulates elements 256 m + 4 j + e with fmaf, then an xor
// butterfly, which every lane finishes with the same bits.
__device__ __forceinline__ float wave_sumsq_bf16(const uint16_t* c, int64_t d, int lane) {
    float acc = 0.0f;
    for (int64_t m = 0; m * 256 < d; ++m) {
        const int64_t i = m * 256 + 4 * lane;
        if (i < d) {
            const u32x2_t p = *(const u32x2_t*)(c + i);
            const float c0 = bf16_lo_to_f32(p[0]), c1 = bf16_hi_to_f32(p[0]);
            const float c2 = bf16_lo_to_f32(p[1]), c3 = bf16_hi_to_f32(p[1]);
            acc = __builtin_fmaf(c0, c0, acc);
            acc = __builtin_fmaf(c1, c1, acc);
            acc = __builtin_fmaf(c2, c2, acc);
            acc = __builtin_fmaf(c3, c3, acc);
        }
    }
    return wave_sum_xor(acc);  // xor butterfly 32, 16, ..., 1
}

__global__ void rvq_csq_kernel(const uint16_t* __restrict__ cb, int64_t rows, int64_t d,
                               float* __restrict__ csq) {
    const int lane = threadIdx.x & 63;
    const int64_t row = (int64_t)blockIdx.x * (blockDim.x / 64) + (threadIdx.x >> 6);
    if (row >= rows) return;
    const float s = wave_sumsq_bf16(cb + row * d, d, lane);
    if (lane == 0) csq[row] = s;
}

hipError_t launch_rvq_csq(const uint16_t* codebooks, int64_t rows, int64_t d, float* csq,
                          hipStream_t stream) {
    const int64_t blocks = (rows + 3) / 4;
    hipLaunchKernelGGL(rvq_csq_kernel, dim3((unsigned)blocks), dim3(256), 0, stream, codebooks,
                       rows, d, csq);
    return hipGetLastError();
}

// recon[b, t, :] = sum over l (in order, from +0) of C_l[code_l[b, t / s_l]].
// One thread per 4 consecutive columns of one row.
__global__ void rvq_decode_kernel(const int32_t* __restrict__ codes, int64_t t, int64_t d,
                                  LevelTable L, const uint16_t* __restrict__ cb, int64_t v,
                                  float* __restrict__ recon, int64_t rows) {
    const int64_t q = d / 4;
    const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= rows * q) return;
    const int64_t row = idx / q, col = (idx % q) * 4;
    const int64_t bb = row / t, tt = row % t;
    float a0 = 0.0f, a1 = 0.0f, a2 = 0.0f, a3 = 0.0f;
    for (int l = 0; l < L.levels; ++l) {
        int32_t k = codes[bb * L.total + L.offset[l] + tt / L.stride[l]];
        k = k < 0 ? 0 : (k >= v ? (int32_t)(v - 1) : k);
        const u32x2_t p = *(const u32x2_t*)(cb + ((int64_t)l * v + k) * d + col);
        a0 = a0 + bf16_lo_to_f32(p[0]);
        a1 = a1 + bf16_hi_to_f32(p[0]);
        a2 = a2 + bf16_lo_to_f32(p[1]);
        a3 = a3 + bf16_hi_to_f32(p[1]);
    }
    f32x4_t o;
    o[0] = a0; o[1] = a1; o[2] = a2; o[3] = a3;
    *(f32x4_t*)(recon + row * d + col) = o;
}

hipError_t launch_rvq_decode(const int32_t* codes, int64_t b, int64_t t, int64_t d,
                             int64_t levels, const int32_t* strides, const uint16_t* codebooks,
                             int64_t v, float* recon, hipStream_t stream) {
    const LevelTable L = make_level_table(t, levels, strides);
    const int64_t rows = b * t;
    const int64_t work = rows * (d / 4);
    hipLaunchKernelGGL(rvq_decode_kernel, dim3((unsigned)((work + 255) / 256)), dim3(256), 0,
                       stream, codes, t, d, L, codebooks, v, recon, rows);
    return hipGetLastError();
}

}  // namespace ncm
