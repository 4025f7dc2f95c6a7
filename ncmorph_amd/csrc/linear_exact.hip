// The bf16 linear in the reference's own arithmetic, bit for bit:
// matmul_bf16_impl (packages/kernels/root.zig:106-142), the emulation of
// oneDNN's brg_matmul:avx512_core_bf16 (PROJECT.md:519, D67).
//
// For each output (t, o): the reduction runs in blocks of
// Kb = min(K, K > 1024 ? 1024 : 512) elements; inside a block, from +0,
//   partial = ftz(fma(x[i + 1], w[i + 1], partial))
//   partial = ftz(fma(x[i], w[i], partial))
// for the pairs (i, i + 1) from the block start, an odd last element alone;
// operands are bf16 values with subnormals flushed (ftz keeps the sign);
// sum += partial after each block (no flush), then sum += bias (a bf16
// value), and the output is round_bf16(sum) (or sum itself in the F32 mode).
//
// One fp32 fma per multiply-add on the VALU, in that order: the MFMA cannot
// reproduce it (its internal summation order differs), so this path exists
// for callers that need the reference's bits (its real-checkpoint logit
// gates), not for speed. A workgroup computes a 64 x 64 output tile, each
// thread a 4 x 4 register block (rows ty + 16 i, columns tx + 16 j); 64-element
// K chunks are staged in LDS as bf16 pairs (x[k], x[k + 1]) packed in 32-bit
// words, [pair][row], so one LDS read gives a thread both elements of a pair.
// Chunks start at multiples of 64 and blocks at multiples of 512, so every
// pair of a chunk lies inside one block.
#include "common.h"
#include "linear.h"

namespace ncm {

namespace {

constexpr int kExTile = 64;   // output rows and columns per workgroup
constexpr int kExChunk = 64;  // K elements per LDS chunk
constexpr int kExPairs = kExChunk / 2;

__device__ __forceinline__ float ftz(float v) { return flush_subnormal(v); }

__global__ __launch_bounds__(256) void linear_exact_kernel(const uint16_t* __restrict__ x,
                                                            const uint16_t* __restrict__ w,
                                                            const uint16_t* __restrict__ bias,
                                                            void* __restrict__ y, int64_t M,
                                                            int64_t K, int64_t N, int out_mode,
                                                            int64_t tiles_n) {
    // +1 column: the staging writes of one pair index by 64 consecutive rows
    // and the reads of 16 consecutive columns land in distinct banks.
    __shared__ uint32_t xs[kExPairs][kExTile + 1];
    __shared__ uint32_t wsh[kExPairs][kExTile + 1];
    const int tid = threadIdx.x;
    const int tx = tid & 15, ty = tid >> 4;
    const int64_t r0 = (int64_t)blockIdx.x / tiles_n * kExTile;
    const int64_t c0 = (int64_t)blockIdx.x % tiles_n * kExTile;
    const int64_t kb = K < (K > 1024 ? 1024 : 512) ? K : (K > 1024 ? 1024 : 512);

    float partial[4][4], sum[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) partial[i][j] = sum[i][j] = 0.0f;

    for (int64_t k0 = 0; k0 < K; k0 += kExChunk) {
        // Stage 64 rows x 32 pairs of each operand (8 pairs per thread).
#pragma unroll
        for (int q = 0; q < (kExTile * kExPairs) / 256; ++q) {
            const int idx = tid + 256 * q;
            const int r = idx / kExPairs, p = idx % kExPairs;
            const int64_t k = k0 + 2 * p;
            uint32_t vx = 0, vw = 0;
            if (r0 + r < M) {
                const uint16_t* row = x + (r0 + r) * K;
                const uint32_t lo = k < K ? row[k] : 0u, hi = k + 1 < K ? row[k + 1] : 0u;
                vx = lo | (hi << 16);
            }
            if (c0 + r < N) {
                const uint16_t* row = w + (c0 + r) * K;
                const uint32_t lo = k < K ? row[k] : 0u, hi = k + 1 < K ? row[k + 1] : 0u;
                vw = lo | (hi << 16);
            }
            xs[p][r] = vx;
            wsh[p][r] = vw;
        }
        __syncthreads();
        const int64_t left = K - k0;
        const int np = left >= kExChunk ? kExPairs : (int)((left + 1) / 2);
        for (int p = 0; p < np; ++p) {
            const int64_t k = k0 + 2 * p;
            float ahi[4], alo[4], bhi[4], blo[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const uint32_t a = xs[p][ty + 16 * i];
                const uint32_t b = wsh[p][tx + 16 * i];
                ahi[i] = ftz(bf16_hi_to_f32(a));
                alo[i] = ftz(bf16_lo_to_f32(a));
                bhi[i] = ftz(bf16_hi_to_f32(b));
                blo[i] = ftz(bf16_lo_to_f32(b));
            }
            if (k + 1 < K) {
#pragma unroll
                for (int i = 0; i < 4; ++i)
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        partial[i][j] = ftz(__builtin_fmaf(ahi[i], bhi[j], partial[i][j]));
                        partial[i][j] = ftz(__builtin_fmaf(alo[i], blo[j], partial[i][j]));
                    }
            } else {
                // The odd last element of the last block.
#pragma unroll
                for (int i = 0; i < 4; ++i)
#pragma unroll
                    for (int j = 0; j < 4; ++j)
                        partial[i][j] = ftz(__builtin_fmaf(alo[i], blo[j], partial[i][j]));
            }
            // End of a block: the pair that reaches a multiple of kb or K.
            if (k + 2 >= K || (k + 2) % kb == 0) {
#pragma unroll
                for (int i = 0; i < 4; ++i)
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        sum[i][j] = sum[i][j] + partial[i][j];
                        partial[i][j] = 0.0f;
                    }
            }
        }
        __syncthreads();
    }

#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int64_t c = c0 + tx + 16 * j;
        if (c >= N) continue;
        const float bv = bias ? __uint_as_float((uint32_t)bias[c] << 16) : 0.0f;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int64_t r = r0 + ty + 16 * i;
            if (r >= M) continue;
            float s = sum[i][j];
            if (bias) s = s + bv;
            const int64_t o = r * N + c;
            if (out_mode == NCM_OUT_F32) {
                ((float*)y)[o] = s;
            } else {
                const uint32_t bits = bf16_bits_rne(s);
                if (out_mode == NCM_OUT_BF16)
                    ((uint16_t*)y)[o] = (uint16_t)bits;
                else
                    ((float*)y)[o] = __uint_as_float(bits << 16);
            }
        }
    }
}

}  // namespace

hipError_t launch_linear_exact(const uint16_t* x, const uint16_t* w, const uint16_t* bias,
                               void* y, int64_t M, int64_t K, int64_t N, int out_mode,
                               hipStream_t stream) {
    if (M <= 0 || N <= 0) return hipSuccess;
    const int64_t tiles_m = (M + kExTile - 1) / kExTile, tiles_n = (N + kExTile - 1) / kExTile;
    if (tiles_m * tiles_n > 0x7FFFFFFF) return hipErrorInvalidValue;
    hipLaunchKernelGGL(linear_exact_kernel, dim3((unsigned)(tiles_m * tiles_n)), dim3(256), 0,
                       stream, x, w, bias, y, M, K, N, out_mode, tiles_n);
    return hipGetLastError();
}

}  // namespace ncm
