// Elementwise bf16 conversions (memory-bound, coalesced, vectorized).
// f32 -> bf16: packages/bf16/root.zig:17-22 (RNE, every NaN -> 0x7FC0),
// optionally followed by the operand flush of packages/kernels/root.zig:124-135.
// bf16 -> f32: packages/bf16/root.zig:25-37 (exact widen).
#include "common.h"
#include "linear.h"

namespace ncm {

__device__ __forceinline__ uint32_t to_bf16(float v, int flush) {
    uint32_t b = bf16_bits_rne(v);
    if (flush && (b & 0x7F80u) == 0) b &= 0x8000u;
    return b;
}

__global__ void bf16_from_f32_kernel(const float* __restrict__ src, uint16_t* __restrict__ dst,
                                     int64_t n, int flush) {
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    const int64_t n4 = n / 4;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n4; i += stride) {
        const f32x4_t v = ((const f32x4_t*)src)[i];
        u32x2_t o;
        o[0] = to_bf16(v[0], flush) | (to_bf16(v[1], flush) << 16);
        o[1] = to_bf16(v[2], flush) | (to_bf16(v[3], flush) << 16);
        ((u32x2_t*)dst)[i] = o;
    }
    for (int64_t i = n4 * 4 + (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride)
        dst[i] = (uint16_t)to_bf16(src[i], flush);
}

__global__ void bf16_from_f32_2d_kernel(const float* __restrict__ src, uint16_t* __restrict__ dst,
                                        int64_t rows, int64_t cols, int64_t ld, int flush) {
    const int64_t total = rows * ld;
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += stride) {
        const int64_t r = i / ld, c = i % ld;
        dst[i] = c < cols ? (uint16_t)to_bf16(src[r * cols + c], flush) : (uint16_t)0;
    }
}

__global__ void bf16_widen_kernel(const uint16_t* __restrict__ src, float* __restrict__ dst,
                                  int64_t n) {
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride)
        dst[i] = __uint_as_float((uint32_t)src[i] << 16);
}

static dim3 grid_for(int64_t work) {
    int64_t blocks = (work + 255) / 256;
    if (blocks > 4096) blocks = 4096;
    if (blocks < 1) blocks = 1;
    return dim3((unsigned)blocks);
}

hipError_t launch_bf16_from_f32(const float* src, uint16_t* dst, int64_t n, int flush,
                                hipStream_t stream) {
    const bool aligned = ((uintptr_t)src % 16 == 0) && ((uintptr_t)dst % 8 == 0);
    if (aligned) {
        hipLaunchKernelGGL(bf16_from_f32_kernel, grid_for(n / 4 + 1), dim3(256), 0, stream, src,
                           dst, n, flush);
    } else {
        hipLaunchKernelGGL(bf16_from_f32_2d_kernel, grid_for(n), dim3(256), 0, stream, src, dst,
                           (int64_t)1, n, n, flush);
    }
    return hipGetLastError();
}

hipError_t launch_bf16_from_f32_2d(const float* src, uint16_t* dst, int64_t rows, int64_t cols,
                                   int64_t ld, int flush, hipStream_t stream) {
    hipLaunchKernelGGL(bf16_from_f32_2d_kernel, grid_for(rows * ld), dim3(256), 0, stream, src,
                       dst, rows, cols, ld, flush);
    return hipGetLastError();
}

hipError_t launch_bf16_widen(const uint16_t* src, float* dst, int64_t n, hipStream_t stream) {
    hipLaunchKernelGGL(bf16_widen_kernel, grid_for(n), dim3(256), 0, stream, src, dst, n);
    return hipGetLastError();
}

}  // namespace ncm
