// Decoder ops around the bf16 linear (packages/kernels/root.zig:150-270,
// src/decoder.zig:168-216): RMSNorm rows with the reference's pinned
// sum-of-squares cascade, and the MLP activation round_bf16(silu_bf16(gate) *
// up). Memory-bound: each kernel reads its inputs and writes its output once.
#include "common.h"
#include "linear.h"

namespace ncm {

// One wavefront per row. The pinned cascade of root.zig:152-227 keeps 4 x 4 x
// 8 accumulators acc[level][r][l]; every (r, l) chain sees the same sequence
// of operations, so lane c < 32 runs chain (r = c / 8, l = c % 8) with its
// four levels in registers, and the merges that cross chains (rows into the
// vector sum, lanes into the scalar sum) run in the reference's order on
// values gathered by shuffles. Every product and sum is a separate fp32 op
// (built with -ffp-contract=off), as in the reference.
// Widths 1024, 2048 and 4096 (the decoder and NCM hidden sizes) hold the
// row in registers for both passes (rms_norm_rows_reg_kernel: 8224 x 4096
// rows measured 53.5 -> 39.0 us, 4096 x 2048 11.95 -> 10.7 us). Other widths
// read the row from global memory twice (the second pass mostly from the
// caches): staging it in LDS measured slower at widths 2048-8192, since the
// 16 KB-per-row stages held the kernel to two workgroups per CU.

// The pinned sum of squares of one row (root.zig:152-227) by one
// wavefront: lane c < 32 runs chain (r = c / 8, l = c % 8) with its four
// levels in registers, and the merges that cross chains run in the
// reference's order on values gathered by shuffles. Every lane returns the
// same bits. xr: the row in global memory or LDS. TWO: each half-wavefront
// runs the 32 chains of its own row (xr: that half's row; live: whether it
// exists) and returns that row's sum.
template <bool TWO = false>
__device__ __forceinline__ float rms_sum_squares(const float* xr, int64_t n, int lane,
                                                 bool live = true) {
    const bool chain = TWO ? live : lane < 32;
    const int base = TWO ? (lane & 32) : 0;
    const int r = (lane >> 3) & 3, l = lane & 7;

    const int64_t vectors = n / 8, groups = vectors / 4;
    int lg = 0;
    for (int64_t lim = 1; lim < groups; lim *= 2) ++lg;
    const int power = lg / 4 > 4 ? lg / 4 : 4;
    const int64_t step = (int64_t)1 << power, mask = step - 1;
    float a0 = 0.0f, a1 = 0.0f, a2 = 0.0f, a3 = 0.0f;
    auto sq = [&](int64_t vi) {
        const float v = chain ? xr[vi * 8 + l] : 0.0f;
        return v * v;
    };
    int64_t g = 0;
    while (g + step <= groups) {
        if (step == 16) {
            // The common case (up to 2^20 elements): the 16 loads of a run
            // issue together, then the chain adds them in order.
            float t[16];
#pragma unroll
            for (int s = 0; s < 16; ++s) t[s] = sq((g + s) * 4 + r);
#pragma unroll
            for (int s = 0; s < 16; ++s) a0 = a0 + t[s];
        } else {
            for (int64_t s = 0; s < step; ++s) a0 = a0 + sq((g + s) * 4 + r);
        }
        g += step;
        a1 = a1 + a0;
        a0 = 0.0f;
        if ((g & (mask << power)) == 0) {
            a2 = a2 + a1;
            a1 = 0.0f;
            if ((g & (mask << (2 * power))) == 0) {
                a3 = a3 + a2;
                a2 = 0.0f;
            }
        }
    }
    for (; g < groups; ++g) a0 = a0 + sq(g * 4 + r);
    a0 = a0 + a1;
    a0 = a0 + a2;
    a0 = a0 + a3;
    if (r == 0)  // vector tail, into row 0's chains
        for (int64_t vi = groups * 4; vi < vectors; ++vi) a0 = a0 + sq(vi);
    // vector_sum[l] = ((acc[0][0][l] + acc[0][1][l]) + acc[0][2][l]) + acc[0][3][l]
    const float r1 = __shfl(a0, base + l + 8, 64), r2 = __shfl(a0, base + l + 16, 64),
                r3 = __shfl(a0, base + l + 24, 64);
    float vs = a0;
    vs = vs + r1;
    vs = vs + r2;
    vs = vs + r3;
    float sum = 0.0f;
    for (int64_t i = vectors * 8; i < n; ++i) {
        const float v = live ? xr[i] : 0.0f;
        sum = sum + v * v;
    }
#pragma unroll
    for (int k = 0; k < 8; ++k) sum = sum + __shfl(vs, base + k, 64);
    return sum;
}

// The output pass of one row by one wavefront, given 1 / rms.
template <int OUT_MODE>
__device__ __forceinline__ void rms_write_row(const float* __restrict__ x,
                                              const float* __restrict__ weight,
                                              void* __restrict__ y, int64_t row, int64_t n,
                                              float inv, int lane) {
    const float* xr = x + row * n;
    // f32 mode (OUT_MODE NCM_OUT_F32, rms_norm, root.zig:226-239):
    // (x * inv) * weight. bf16 mode: round_bf16(round_bf16(x * inv) *
    // round_bf16(weight)) (root.zig:250-252).
    auto out1 = [&](int64_t i, float v, float wv) {
        if (OUT_MODE == NCM_OUT_F32) {
            const float normalized = v * inv;
            ((float*)y)[row * n + i] = normalized * wv;
            return;
        }
        const float normalized = __uint_as_float(bf16_bits_rne(v * inv) << 16);
        const uint32_t bits = bf16_bits_rne(normalized * __uint_as_float(bf16_bits_rne(wv) << 16));
        if (OUT_MODE == NCM_OUT_BF16)
            ((uint16_t*)y)[row * n + i] = (uint16_t)bits;
        else
            ((float*)y)[row * n + i] = __uint_as_float(bits << 16);
    };
    if (OUT_MODE == NCM_OUT_F32) {
        for (int64_t i = lane; i < n; i += 64) out1(i, xr[i], weight[i]);
    } else if ((n & 3) == 0) {
        // Four elements per lane and step: one 8-byte (bf16) or 16-byte
        // (bf16 values as fp32) store when y is aligned for it.
        const bool yvec = ((uintptr_t)y & (OUT_MODE == NCM_OUT_BF16 ? 7 : 15)) == 0;
        auto emit = [&](int64_t i, const f32x4_t v, const f32x4_t wv) {
            // The same roundings two elements per v_cvt_pk_bf16_f32; the NaN
            // rule on the stored one (a NaN stays a NaN through the product).
            uint32_t bits[4];
#pragma unroll
            for (int e = 0; e < 4; e += 2) {
                const uint32_t nb = bf16x2_rne(v[e] * inv, v[e + 1] * inv);
                const uint32_t wb = bf16x2_rne(wv[e], wv[e + 1]);
                const uint32_t r = bf16x2_bits_rne(
                    __uint_as_float(nb << 16) * __uint_as_float(wb << 16),
                    __uint_as_float(nb & 0xFFFF0000u) * __uint_as_float(wb & 0xFFFF0000u));
                bits[e] = r & 0xFFFFu;
                bits[e + 1] = r >> 16;
            }
            if (!yvec) {
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    if (OUT_MODE == NCM_OUT_BF16)
                        ((uint16_t*)y)[row * n + i + e] = (uint16_t)bits[e];
                    else
                        ((float*)y)[row * n + i + e] = __uint_as_float(bits[e] << 16);
                }
            } else if (OUT_MODE == NCM_OUT_BF16) {
                u32x2_t o;
                o[0] = bits[0] | (bits[1] << 16);
                o[1] = bits[2] | (bits[3] << 16);
                *(u32x2_t*)((uint16_t*)y + row * n + i) = o;
            } else {
                f32x4_t o;
#pragma unroll
                for (int e = 0; e < 4; ++e) o[e] = __uint_as_float(bits[e] << 16);
                *(f32x4_t*)((float*)y + row * n + i) = o;
            }
        };
        // Four steps' loads (x from LDS or global, the weight from global)
        // issued together; lanes past the row load its last chunk and store
        // nothing.
        for (int64_t base = 4 * lane; base < n; base += 4 * 256) {
            f32x4_t vq[4], wq[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int64_t i = base + 256 * j < n ? base + 256 * j : n - 4;
                vq[j] = *(const f32x4_t*)(xr + i);
                wq[j] = *(const f32x4_t*)(weight + i);
            }
#pragma unroll
            for (int j = 0; j < 4; ++j)
                if (base + 256 * j < n) emit(base + 256 * j, vq[j], wq[j]);
        }
    } else {
        for (int64_t i = lane; i < n; i += 64) out1(i, xr[i], weight[i]);
    }
}

// Widths 64 NR (NR = 16, 32, 64: 1024 to 4096 elements): one row per
// wavefront, read once and held in registers (lane j holds x[64 i + j] in
// v[i]) for both passes, instead of the second pass reading the row again.
// The pinned cascade above, on the same chains: chain c = lane c < 32 takes
// x[32 q + c] as its q-th element, which is v[q / 2] of lane c for even q
// and of lane c + 32 for odd q (a permlane32 swap), in the same order with
// the same operations, so the sum has the same bits.
constexpr int rms_ilog2_ceil(int v) {
    int lg = 0;
    while ((1 << lg) < v) ++lg;
    return lg;
}

template <int NR>
__device__ __forceinline__ float rms_sum_squares_reg(const float (&v)[NR], int lane) {
    constexpr int groups = 2 * NR;
    constexpr int lg = rms_ilog2_ceil(groups);
    constexpr int power = lg / 4 > 4 ? lg / 4 : 4;
    constexpr int step = 1 << power, mask = step - 1;
    const int l = lane & 7;
    auto elem = [&](int q) {
        return (q & 1) ? __uint_as_float(swap32(__float_as_uint(v[q >> 1]))[1]) : v[q >> 1];
    };
    float a0 = 0.0f, a1 = 0.0f, a2 = 0.0f, a3 = 0.0f;
    int g = 0;
#pragma unroll
    for (int run = 0; run < groups / step; ++run) {
        // One run's swaps at a time (all of them at once would double the
        // registers).
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int s = 0; s < step; ++s) {
            const float e = elem(run * step + s);
            a0 = a0 + e * e;
        }
        g += step;
        a1 = a1 + a0;
        a0 = 0.0f;
        if ((g & (mask << power)) == 0) {
            a2 = a2 + a1;
            a1 = 0.0f;
            if ((g & (mask << (2 * power))) == 0) {
                a3 = a3 + a2;
                a2 = 0.0f;
            }
        }
    }
#pragma unroll
    for (int q = (groups / step) * step; q < groups; ++q) {
        const float e = elem(q);
        a0 = a0 + e * e;
    }
    a0 = a0 + a1;
    a0 = a0 + a2;
    a0 = a0 + a3;
    // The merges of rms_sum_squares (no vector or scalar tail at these widths).
    const float r1 = __shfl(a0, l + 8, 64), r2 = __shfl(a0, l + 16, 64),
                r3 = __shfl(a0, l + 24, 64);
    float vs = a0;
    vs = vs + r1;
    vs = vs + r2;
    vs = vs + r3;
    float sum = 0.0f;
#pragma unroll
    for (int k = 0; k < 8; ++k) sum = sum + __shfl(vs, k, 64);
    return sum;
}

template <int OUT_MODE, int NR>
__global__ __launch_bounds__(256) void rms_norm_rows_reg_kernel(const float* __restrict__ x,
                                                                const float* __restrict__ weight,
                                                                void* __restrict__ y,
                                                                int64_t rows, float epsilon) {
    static_assert(NR % 2 == 0, "element pairs");
    constexpr int64_t n = 64 * NR;
    const int lane = threadIdx.x & 63;
    const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= rows) return;
    // Buffer loads: the row's base in the resource, the lane's offset in one
    // VGPR, each 256-byte step in the scalar offset.
    const __amdgpu_buffer_rsrc_t rx = make_rsrc(x + row * n, (uint32_t)(n * 4));
    const __amdgpu_buffer_rsrc_t rw = make_rsrc(weight, (uint32_t)(n * 4));
    const uint32_t lo = 4u * (uint32_t)lane;
    float v[NR];
#pragma unroll
    for (int i = 0; i < NR; ++i)
        v[i] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rx, lo, 256 * i, 0));
    const float sum = rms_sum_squares_reg<NR>(v, lane);
    const float mean = sum / (float)n;
    const float inv = 1.0f / sqrtf(mean + epsilon);
    // The output pass of rms_write_row: the same operations, two elements
    // (v[i], v[i + 1]) per rounding instruction.
#pragma unroll
    for (int i = 0; i < NR; i += 2) {
        if (i % 8 == 0) __builtin_amdgcn_sched_barrier(0);
        const float w0 = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rw, lo, 256 * i, 0));
        const float w1 =
            __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rw, lo, 256 * (i + 1), 0));
        const int64_t e0 = row * n + 64 * i + lane, e1 = e0 + 64;
        if (OUT_MODE == NCM_OUT_F32) {
            const float n0 = v[i] * inv, n1 = v[i + 1] * inv;
            ((float*)y)[e0] = n0 * w0;
            ((float*)y)[e1] = n1 * w1;
            continue;
        }
        const uint32_t nb = bf16x2_rne(v[i] * inv, v[i + 1] * inv);
        const uint32_t wb = bf16x2_rne(w0, w1);
        const uint32_t r = bf16x2_bits_rne(
            __uint_as_float(nb << 16) * __uint_as_float(wb << 16),
            __uint_as_float(nb & 0xFFFF0000u) * __uint_as_float(wb & 0xFFFF0000u));
        if (OUT_MODE == NCM_OUT_BF16) {
            ((uint16_t*)y)[e0] = (uint16_t)(r & 0xFFFFu);
            ((uint16_t*)y)[e1] = (uint16_t)(r >> 16);
        } else {
            ((float*)y)[e0] = __uint_as_float(r << 16);
            ((float*)y)[e1] = __uint_as_float(r & 0xFFFF0000u);
        }
    }
}

// TWO: two rows per wavefront (the first in lanes 0-31's chains, the second
// in lanes 32-63's), then the output pass of each in turn by the whole
// wavefront: used when the rows outnumber the wavefronts the chip holds at
// once, where one row per wavefront would leave the last few rows a second
// round of their own.
template <int OUT_MODE, bool TWO>
__global__ __launch_bounds__(256) void rms_norm_rows_kernel(const float* __restrict__ x,
                                                            const float* __restrict__ weight,
                                                            void* __restrict__ y, int64_t rows,
                                                            int64_t n, float epsilon) {
    const int lane = threadIdx.x & 63;
    const int64_t wrow = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    const int64_t row0 = TWO ? 2 * wrow : wrow;
    if (row0 >= rows) return;
    if constexpr (TWO) {
        const int h = lane >> 5;
        const bool live = row0 + h < rows;
        const float sum =
            rms_sum_squares<true>(x + (row0 + (live ? h : 0)) * n, n, lane, live);
        const float mean = sum / (float)n;
        const float inv = 1.0f / sqrtf(mean + epsilon);
        const float inv0 = __shfl(inv, 0, 64), inv1 = __shfl(inv, 32, 64);
        rms_write_row<OUT_MODE>(x, weight, y, row0, n, inv0, lane);
        if (row0 + 1 < rows) rms_write_row<OUT_MODE>(x, weight, y, row0 + 1, n, inv1, lane);
    } else {
        const float sum = rms_sum_squares(x + row0 * n, n, lane);
        const float mean = sum / (float)n;
        const float inv = 1.0f / sqrtf(mean + epsilon);
        rms_write_row<OUT_MODE>(x, weight, y, row0, n, inv, lane);
    }
}

// round_bf16(round_bf16(g / (1 + exp(-g))) * up) (root.zig:265-270,
// src/decoder.zig:210-211), four elements per thread (16-byte loads when the
// four are in range and aligned).
template <int OUT_MODE>
__global__ __launch_bounds__(256) void silu_mul_kernel(const float* __restrict__ gate,
                                                       const float* __restrict__ up,
                                                       void* __restrict__ y, int64_t n) {
    if (OUT_MODE == NCM_OUT_F32) {
        // f32 mode: silu(g) = g * (1 / (1 + exp(-g))) (root.zig:255-261), then
        // the product with up unrounded (src/decoder.zig:210-211).
        const int64_t i0 = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) * 4;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int64_t i = i0 + e;
            if (i >= n) break;
            const float v = gate[i];
            const float sigmoid = 1.0f / (1.0f + expf(-v));
            const float a = v * sigmoid;
            ((float*)y)[i] = up ? a * up[i] : a;
        }
        return;
    }
    auto act = [](float v, float u) {
        const float a = __uint_as_float(bf16_bits_rne(v / (1.0f + expf(-v))) << 16);
        return bf16_bits_rne(a * u);
    };
    const int64_t i0 = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) * 4;
    if (i0 >= n) return;
    const bool vec = i0 + 4 <= n && ((uintptr_t)gate & 15) == 0 && (!up || ((uintptr_t)up & 15) == 0);
    uint32_t b[4];
    if (vec) {
        const f32x4_t g = *(const f32x4_t*)(gate + i0);
        f32x4_t u = {1.0f, 1.0f, 1.0f, 1.0f};
        if (up) u = *(const f32x4_t*)(up + i0);
        // act() two elements at a time: the roundings per v_cvt_pk_bf16_f32,
        // the NaN rule on the stored one (a NaN stays a NaN through a * u).
#pragma unroll
        for (int e = 0; e < 4; e += 2) {
            const uint32_t a = bf16x2_rne(g[e] / (1.0f + expf(-g[e])),
                                          g[e + 1] / (1.0f + expf(-g[e + 1])));
            const uint32_t r = bf16x2_bits_rne(__uint_as_float(a << 16) * u[e],
                                               __uint_as_float(a & 0xFFFF0000u) * u[e + 1]);
            b[e] = r & 0xFFFFu;
            b[e + 1] = r >> 16;
        }
        if (OUT_MODE == NCM_OUT_BF16 && ((uintptr_t)y & 7) == 0) {
            u32x2_t o;
            o[0] = b[0] | (b[1] << 16);
            o[1] = b[2] | (b[3] << 16);
            *(u32x2_t*)((uint16_t*)y + i0) = o;
            return;
        }
        if (OUT_MODE != NCM_OUT_BF16 && ((uintptr_t)y & 15) == 0) {
            u32x4_t o;
#pragma unroll
            for (int e = 0; e < 4; ++e) o[e] = b[e] << 16;
            *(u32x4_t*)((float*)y + i0) = o;
            return;
        }
    } else {
#pragma unroll
        for (int e = 0; e < 4; ++e)
            b[e] = i0 + e < n ? act(gate[i0 + e], up ? up[i0 + e] : 1.0f) : 0u;
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        if (i0 + e >= n) break;
        if (OUT_MODE == NCM_OUT_BF16)
            ((uint16_t*)y)[i0 + e] = (uint16_t)b[e];
        else
            ((float*)y)[i0 + e] = __uint_as_float(b[e] << 16);
    }
}

// rotate_head in bf16 mode (root.zig:615-634) over every head of every row,
// in place on bf16 bits: row r, head h occupies x[r * row_stride + h * hd ..
// + hd); its table row is position r % seq_len of cosine/sine [seq_len, hd].
// Each table entry, product and sum is rounded to bf16, in the reference's
// order; one thread per (row, head, i < hd / 2) pair of elements.
__global__ __launch_bounds__(256) void rope_rotate_kernel(uint16_t* __restrict__ x, int64_t rows,
                                                          int64_t row_stride, int heads, int hd,
                                                          int64_t seq_len,
                                                          const float* __restrict__ cosine,
                                                          const float* __restrict__ sine) {
    const int half = hd >> 1;
    const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= rows * heads * half) return;
    const int i = (int)(idx % half);
    const int64_t rh = idx / half;
    const int h = (int)(rh % heads);
    const int64_t r = rh / heads;
    const int64_t pos = r % seq_len;
    auto rb = [](float v) { return __uint_as_float(bf16_bits_rne(v) << 16); };
    uint16_t* e = x + r * row_stride + (int64_t)h * hd + i;
    const float first = __uint_as_float((uint32_t)e[0] << 16);
    const float second = __uint_as_float((uint32_t)e[half] << 16);
    const float* ct = cosine + pos * hd + i;
    const float* st = sine + pos * hd + i;
    const float cos_first = rb(ct[0]), sin_first = rb(st[0]);
    const float cos_second = rb(ct[half]), sin_second = rb(st[half]);
    const float left = rb(first * cos_first);
    const float right = rb(-second * sin_first);
    const float right2 = rb(first * sin_second);
    const float left2 = rb(second * cos_second);
    e[0] = (uint16_t)bf16_bits_rne(left + right);
    e[half] = (uint16_t)bf16_bits_rne(left2 + right2);
}

// The same rotation, four consecutive pairs per thread (8-byte element and
// 16-byte table loads, 32-bit index arithmetic) for a batch of hb heads of
// one row (hb 8, or 1 when the launch would otherwise have too few threads
// to fill the chip): the table values of a (row, pair group) are loaded and
// rounded once per batch and serve its heads. The roundings run two values
// per v_cvt_pk_bf16_f32 (the bits of bf16_bits_rne for every non-NaN value;
// a NaN stays a NaN up to the final rounding, which maps it to 0x7FC0 as
// bf16_bits_rne does). hd % 8 == 0, row_stride % 4 == 0, x 8-byte and the
// tables 16-byte aligned, rows * heads * hd / 8 < 2^31.
constexpr int kRopeHeadBatch = 8;
__global__ __launch_bounds__(256) void rope_rotate4_kernel(uint16_t* __restrict__ x, int rows,
                                                           int64_t row_stride, int heads, int hd,
                                                           int seq_len,
                                                           const float* __restrict__ cosine,
                                                           const float* __restrict__ sine,
                                                           int hb) {
    const int half = hd >> 1, groups = half >> 2;
    const int nbatch = (heads + hb - 1) / hb;
    const int64_t idx64 = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx64 >= (int64_t)rows * nbatch * groups) return;
    const int idx = (int)idx64;  // < 2^31 (checked by the launcher)
    const int i = 4 * (idx % groups);
    const int rb = idx / groups;
    const int h0 = hb * (rb % nbatch);
    const int h1 = h0 + hb < heads ? h0 + hb : heads;  // the batch's end
    const int r = rb / nbatch;
    const int pos = r % seq_len;
    const float* ct = cosine + (int64_t)pos * hd + i;
    const float* st = sine + (int64_t)pos * hd + i;
    const f32x4_t c1 = *(const f32x4_t*)ct, s1 = *(const f32x4_t*)st;
    const f32x4_t c2 = *(const f32x4_t*)(ct + half), s2 = *(const f32x4_t*)(st + half);
    auto lo = [](uint32_t p) { return __uint_as_float(p << 16); };
    auto hi = [](uint32_t p) { return __uint_as_float(p & 0xFFFF0000u); };
    // rb(table) for elements (0, 1) and (2, 3).
    uint32_t tc1[2], ts1[2], tc2[2], ts2[2];
#pragma unroll
    for (int k = 0; k < 2; ++k) {
        tc1[k] = bf16x2_rne(c1[2 * k], c1[2 * k + 1]);
        ts1[k] = bf16x2_rne(s1[2 * k], s1[2 * k + 1]);
        tc2[k] = bf16x2_rne(c2[2 * k], c2[2 * k + 1]);
        ts2[k] = bf16x2_rne(s2[2 * k], s2[2 * k + 1]);
    }
    uint16_t* row = x + (int64_t)r * row_stride + i;
    // The batch's loads issued together, then its rotations and stores.
    u32x2_t fa[kRopeHeadBatch], fb[kRopeHeadBatch];
#pragma unroll
    for (int b = 0; b < kRopeHeadBatch; ++b) {
        if (h0 + b < h1) {
            const uint16_t* e = row + (int64_t)(h0 + b) * hd;
            fa[b] = *(const u32x2_t*)e;
            fb[b] = *(const u32x2_t*)(e + half);
        }
    }
#pragma unroll
    for (int b = 0; b < kRopeHeadBatch; ++b) {
        if (h0 + b >= h1) break;
        uint16_t* e = row + (int64_t)(h0 + b) * hd;
        u32x2_t w1, w2;
#pragma unroll
        for (int k = 0; k < 2; ++k) {
            const uint32_t wa = fa[b][k], wb = fb[b][k];
            const float f0 = lo(wa), f1 = hi(wa), s0 = lo(wb), s1v = hi(wb);
            const uint32_t left = bf16x2_rne(f0 * lo(tc1[k]), f1 * hi(tc1[k]));
            const uint32_t right = bf16x2_rne(-s0 * lo(ts1[k]), -s1v * hi(ts1[k]));
            const uint32_t right2 = bf16x2_rne(f0 * lo(ts2[k]), f1 * hi(ts2[k]));
            const uint32_t left2 = bf16x2_rne(s0 * lo(tc2[k]), s1v * hi(tc2[k]));
            w1[k] = bf16x2_bits_rne(lo(left) + lo(right), hi(left) + hi(right));
            w2[k] = bf16x2_bits_rne(lo(left2) + lo(right2), hi(left2) + hi(right2));
        }
        *(u32x2_t*)e = w1;
        *(u32x2_t*)(e + half) = w2;
    }
}

hipError_t launch_rope_rotate(uint16_t* x, int64_t rows, int64_t row_stride, int heads, int hd,
                              int64_t seq_len, const float* cosine, const float* sine,
                              hipStream_t stream) {
    // Batches of 8 heads when one head per thread would give at least 2^20
    // threads, else one head per thread.
    const int hb = rows * heads * (hd / 8) >= ((int64_t)1 << 20) ? kRopeHeadBatch : 1;
    const int64_t n4 = rows * ((heads + hb - 1) / hb) * (hd / 8);
    if (hd % 8 == 0 && row_stride % 4 == 0 && ((uintptr_t)x & 7) == 0 &&
        ((uintptr_t)cosine & 15) == 0 && ((uintptr_t)sine & 15) == 0 && n4 < ((int64_t)1 << 31) &&
        seq_len < ((int64_t)1 << 31)) {
        hipLaunchKernelGGL(rope_rotate4_kernel, dim3((unsigned)((n4 + 255) / 256)), dim3(256), 0,
                           stream, x, (int)rows, row_stride, heads, hd, (int)seq_len, cosine,
                           sine, hb);
        return hipGetLastError();
    }
    const int64_t n = rows * heads * (hd / 2);
    hipLaunchKernelGGL(rope_rotate_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, stream,
                       x, rows, row_stride, heads, hd, seq_len, cosine, sine);
    return hipGetLastError();
}

// QK-norm of the bf16 attention (root.zig:501-530): rms_norm_bf16 of every
// head_dim-wide head of the q (or k) columns, in place on bf16 bits, before
// the rotation. One wavefront per (row, head); the head is widened into LDS
// and reduced with the pinned cascade, as rms_norm_bf16 does for a vector of
// head_dim values.
__global__ __launch_bounds__(256) void qk_norm_kernel(uint16_t* __restrict__ x, int64_t rows,
                                                      int64_t row_stride, int heads, int hd,
                                                      const float* __restrict__ weight,
                                                      float epsilon) {
    __shared__ float stage[4][256];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int64_t item = (int64_t)blockIdx.x * 4 + wave;
    if (item >= rows * heads) return;
    const int64_t r = item / heads;
    const int h = (int)(item % heads);
    uint16_t* e = x + r * row_stride + (int64_t)h * hd;
    float* sr = stage[wave];
    for (int i = lane; i < hd; i += 64) sr[i] = __uint_as_float((uint32_t)e[i] << 16);
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    const float sum = rms_sum_squares(sr, hd, lane);
    const float mean = sum / (float)hd;
    const float inv = 1.0f / sqrtf(mean + epsilon);
    for (int i = lane; i < hd; i += 64) {
        const float normalized = __uint_as_float(bf16_bits_rne(sr[i] * inv) << 16);
        e[i] = (uint16_t)bf16_bits_rne(normalized *
                                       __uint_as_float(bf16_bits_rne(weight[i]) << 16));
    }
}

hipError_t launch_qk_norm(uint16_t* x, int64_t rows, int64_t row_stride, int heads, int hd,
                          const float* weight, float epsilon, hipStream_t stream) {
    if (hd > 256) return hipErrorInvalidValue;
    const int64_t items = rows * heads;
    hipLaunchKernelGGL(qk_norm_kernel, dim3((unsigned)((items + 3) / 4)), dim3(256), 0, stream, x,
                       rows, row_stride, heads, hd, weight, epsilon);
    return hipGetLastError();
}

// y = round_bf16(y + bias[column]) in place over [rows, n]: the bias of
// rms_norm_rows_with_bias (src/ncm_norm.zig:22-49) in bf16 mode, on bf16 bits
// (BITS) or on floats holding bf16 values.
template <bool BITS>
__global__ __launch_bounds__(256) void bias_round_kernel(void* __restrict__ y,
                                                         const float* __restrict__ bias,
                                                         int64_t rows, int64_t n) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= rows * n) return;
    const float b = bias[i % n];
    if (BITS) {
        uint16_t* p = (uint16_t*)y + i;
        *p = (uint16_t)bf16_bits_rne(__uint_as_float((uint32_t)*p << 16) + b);
    } else {
        float* p = (float*)y + i;
        *p = __uint_as_float(bf16_bits_rne(*p + b) << 16);
    }
}

hipError_t launch_bias_round(void* y, const float* bias, int64_t rows, int64_t n, bool bits,
                             hipStream_t stream) {
    const int64_t total = rows * n;
    const dim3 grid((unsigned)((total + 255) / 256));
    if (bits)
        hipLaunchKernelGGL(bias_round_kernel<true>, grid, dim3(256), 0, stream, y, bias, rows, n);
    else
        hipLaunchKernelGGL(bias_round_kernel<false>, grid, dim3(256), 0, stream, y, bias, rows, n);
    return hipGetLastError();
}

template <int OUT_MODE>
static hipError_t launch_rms_t(const float* x, const float* weight, void* y, int64_t rows,
                               int64_t n, float epsilon, hipStream_t stream) {
    const dim3 grid1((unsigned)((rows + 3) / 4));
    switch (n) {
        case 1024:
            hipLaunchKernelGGL((rms_norm_rows_reg_kernel<OUT_MODE, 16>), grid1, dim3(256), 0,
                               stream, x, weight, y, rows, epsilon);
            return hipGetLastError();
        case 2048:
            hipLaunchKernelGGL((rms_norm_rows_reg_kernel<OUT_MODE, 32>), grid1, dim3(256), 0,
                               stream, x, weight, y, rows, epsilon);
            return hipGetLastError();
        case 4096:
            hipLaunchKernelGGL((rms_norm_rows_reg_kernel<OUT_MODE, 64>), grid1, dim3(256), 0,
                               stream, x, weight, y, rows, epsilon);
            return hipGetLastError();
        default:
            break;
    }
    // Wavefronts resident at once: 8 per SIMD on 256 CUs.
    constexpr int64_t kResidentWaves = 256 * 4 * 8;
    if (rows > kResidentWaves)
        hipLaunchKernelGGL((rms_norm_rows_kernel<OUT_MODE, true>),
                           dim3((unsigned)((rows + 7) / 8)), dim3(256), 0, stream, x, weight, y,
                           rows, n, epsilon);
    else
        hipLaunchKernelGGL((rms_norm_rows_kernel<OUT_MODE, false>),
                           dim3((unsigned)((rows + 3) / 4)), dim3(256), 0, stream, x, weight, y,
                           rows, n, epsilon);
    return hipGetLastError();
}

hipError_t launch_rms_norm_rows(const float* x, const float* weight, void* y, int64_t rows,
                                int64_t n, float epsilon, int out_mode, hipStream_t stream) {
    if (out_mode == NCM_OUT_F32)
        return launch_rms_t<NCM_OUT_F32>(x, weight, y, rows, n, epsilon, stream);
    if (out_mode == NCM_OUT_BF16)
        return launch_rms_t<NCM_OUT_BF16>(x, weight, y, rows, n, epsilon, stream);
    return launch_rms_t<NCM_OUT_BF16_F32>(x, weight, y, rows, n, epsilon, stream);
}

hipError_t launch_silu_mul(const float* gate, const float* up, void* y, int64_t n, int out_mode,
                           hipStream_t stream) {
    const dim3 grid((unsigned)((n + 1023) / 1024));
    if (out_mode == NCM_OUT_F32)
        hipLaunchKernelGGL(silu_mul_kernel<NCM_OUT_F32>, grid, dim3(256), 0, stream, gate, up, y,
                           n);
    else if (out_mode == NCM_OUT_BF16)
        hipLaunchKernelGGL(silu_mul_kernel<NCM_OUT_BF16>, grid, dim3(256), 0, stream, gate, up, y,
                           n);
    else
        hipLaunchKernelGGL(silu_mul_kernel<NCM_OUT_BF16_F32>, grid, dim3(256), 0, stream, gate,
                           up, y, n);
    return hipGetLastError();
}

}  // namespace ncm
