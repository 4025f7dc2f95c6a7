// The last R (<= 64) rows of a bf16 linear whose 256 x 256 tiles would spend
// a whole extra round of the chip on them. With M = 256 q + R, the row tile
// q holds R valid rows, and when its tiles_n tiles push the tile count past a
// multiple of the CU count, every CU waits for a round that does R / 256 of
// a round's work (the NCM step's 8224 = 32 x 256 + 32 positions: the down
// projection's 528 tiles take three rounds for 2.06 rounds of work). The
// host launches the tile kernel on the first 256 q rows and this kernel on
// the rest.
//
// A skinny product: workgroup b takes 16 output columns (SwiGLU: 16
// features, i.e. their 16 gate and 16 up weight rows) of all R rows over the
// whole K; its 8 wavefronts take one eighth of K each, in 128-element steps
// of v_mfma_f32_16x16x32_bf16 (A = x rows, B = weight rows; MFMA i of a
// step covers k = 32 i .. 32 i + 31, lane group g holding 32 i + 8 g .. + 7,
// so a weight load instruction in that layout reads 64 contiguous bytes of
// 16 rows, straight into registers), and the eight partial sums are added in
// wavefront order through LDS. The x rows, which every workgroup reads (from
// the L2), are loaded 4 rows x 256 contiguous bytes per instruction instead
// (a 16-row x 64-byte instruction touches 16 cache lines and uses half of
// each: the q|k|v tail of the NCM step measured 24.8 -> 15.0 us with
// contiguous x loads alone), written to the wavefront's own LDS region and
// read back as the same A fragments, so every MFMA sees the operands it saw
// before. The epilogue is the tile
// kernels' own: bias, bf16 rounding, residual add (linear_kernel) or
// swiglu_bits2 (linear_pair_kernel). Every output is the same function of
// its row of x and its weight row(s) wherever the row sits in the batch, but
// the fp32 sum runs in another order than the tile kernels', so a tail row
// can differ from the value a 256-row tile would give in the last bits (both
// within the bound of any RNE fp32 summation order).
#include "common.h"
#include "linear.h"

namespace ncm {

namespace {

constexpr int kTailWaves = 8;
constexpr int kTailStepK = 128;  // k per step: 32 per lane group (64 bytes)
constexpr int64_t kTailMaxRows = 64;
constexpr int64_t kTailKMultiple = kTailWaves * 2 * kTailStepK;  // two-step unroll per wave

template <int RB, bool SWIGLU>
struct TailBuf {
    u32x4_t g[4];               // weight rows (SwiGLU: gate rows)
    u32x4_t u[SWIGLU ? 4 : 1];  // SwiGLU: up rows
    u32x4_t a[4 * RB];          // x: load j holds rows 4 j .. 4 j + 3 (16 lanes each)
};

// LDS bytes of the x staging: per wavefront 16 RB rows of one step (256
// bytes each; 16-byte chunk c of row r stored at chunk c ^ (r % 16)).
template <int RB>
constexpr int tail_lds_bytes() {
    return kTailWaves * 16 * RB * kTailStepK * 2;
}

template <int RB, bool SWIGLU, int OUT_MODE, bool HAS_BIAS, bool HAS_RES>
__global__ __launch_bounds__(64 * kTailWaves) void linear_tail_kernel(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ w,
    const uint16_t* __restrict__ bias, const float* residual, void* y, int64_t R, int64_t K,
    int64_t N) {
    constexpr int NACC = SWIGLU ? 2 : 1;
    // x staging during the main loop, then the partial sums (which fit in it).
    extern __shared__ __attribute__((aligned(16))) char tail_lds[];
    static_assert((kTailWaves - 1) * NACC * RB * 64 * 16 <= tail_lds_bytes<RB>(), "partials");
    auto part = reinterpret_cast<f32x4_t(*)[NACC * RB][64]>(tail_lds);
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int r16 = lane & 15, grp = lane >> 4;
    // First output column (SwiGLU: feature) of the workgroup and its first
    // weight row: SwiGLU rows are interleaved in groups of 32 (gate rows
    // 64 (f / 32) + f % 32, up rows 32 further), so the 16 features' gate
    // rows are wr0 .. wr0 + 15 and their up rows wr0 + 32 .. wr0 + 47.
    const int64_t c0 = (int64_t)blockIdx.x * 16;
    const int64_t wr0 = SWIGLU ? 64 * (c0 / 32) + c0 % 32 : c0;
    const __amdgpu_buffer_rsrc_t rsw =
        make_rsrc(w + wr0 * K, (uint32_t)((SWIGLU ? 48 : 16) * K * 2));
    // Rows >= R lie past the resource: they load as zero.
    const __amdgpu_buffer_rsrc_t rsx = make_rsrc(x, (uint32_t)(R * K * 2));
    const int64_t kq = K / kTailWaves;
    const uint32_t kb0 = (uint32_t)((wave * kq + 8 * grp) * 2);
    const uint32_t goff = (uint32_t)(r16 * K * 2) + kb0;
    const uint32_t uoff = (uint32_t)((32 + r16) * K * 2) + kb0;
    // x load j: row 4 j + lane / 16, 16-byte chunk lane % 16 of the step.
    const uint32_t xoff = (uint32_t)(((lane >> 4) * K + wave * kq + 8 * r16) * 2);
    char* xs = tail_lds + wave * (16 * RB * kTailStepK * 2);

    // A step past the end loads from outside both resources (zeros, no
    // memory traffic), so every iteration issues the same loads and the
    // waits before each step's MFMAs count only that step's loads.
    const int steps = (int)(kq / kTailStepK);  // even (K % kTailKMultiple == 0)
    auto load = [&](TailBuf<RB, SWIGLU>& b, int step) {
        const uint32_t kb = step < steps ? (uint32_t)step * (kTailStepK * 2) : kOobOffset;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            b.g[i] = buffer_load_b128(rsw, goff + kb + 64 * i);
            if (SWIGLU) b.u[i] = buffer_load_b128(rsw, uoff + kb + 64 * i);
        }
#pragma unroll
        for (int j = 0; j < 4 * RB; ++j)
            b.a[j] = buffer_load_b128(rsx, xoff + (uint32_t)(4 * j * K * 2) + kb);
    };
    f32x4_t acc[NACC][RB];
#pragma unroll
    for (int a = 0; a < NACC; ++a)
#pragma unroll
        for (int rb = 0; rb < RB; ++rb) acc[a][rb] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
    auto compute = [&](const TailBuf<RB, SWIGLU>& b) {
        // The step's x rows into this wavefront's LDS region, then the A
        // fragments (row 16 rb + r16, chunk 4 i + grp) back out.
#pragma unroll
        for (int j = 0; j < 4 * RB; ++j) {
            const int row = 4 * j + grp;
            *(u32x4_t*)(xs + row * 256 + ((r16 ^ (row & 15)) << 4)) = b.a[j];
        }
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        u32x4_t af[RB][4];
#pragma unroll
        for (int rb = 0; rb < RB; ++rb)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int row = 16 * rb + r16;
                af[rb][i] = *(const u32x4_t*)(xs + row * 256 + (((4 * i + grp) ^ r16) << 4));
            }
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int rb = 0; rb < RB; ++rb) {
                acc[0][rb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                    __builtin_bit_cast(bf16x8_t, af[rb][i]), __builtin_bit_cast(bf16x8_t, b.g[i]),
                    acc[0][rb], 0, 0, 0);
                if (SWIGLU)
                    acc[NACC - 1][rb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                        __builtin_bit_cast(bf16x8_t, af[rb][i]),
                        __builtin_bit_cast(bf16x8_t, b.u[i]), acc[NACC - 1][rb], 0, 0, 0);
            }
    };

    // Two register stages: the next step's loads are issued before this
    // step's MFMAs (the scheduling barriers keep that order) and fly while
    // they run.
    TailBuf<RB, SWIGLU> b0, b1;
    load(b0, 0);
    for (int s = 0; s < steps; s += 2) {
        load(b1, s + 1);
        __builtin_amdgcn_sched_barrier(0);
        compute(b0);
        __builtin_amdgcn_sched_barrier(0);
        load(b0, s + 2);
        __builtin_amdgcn_sched_barrier(0);
        compute(b1);
        __builtin_amdgcn_sched_barrier(0);
    }

    // Partial sums of wavefronts 1 .. 7 to LDS (over the x staging, once
    // every wavefront is past its last step); wavefront 0 adds them in
    // order and runs the epilogue.
    __syncthreads();
    if (wave > 0) {
#pragma unroll
        for (int a = 0; a < NACC; ++a)
#pragma unroll
            for (int rb = 0; rb < RB; ++rb) part[wave - 1][a * RB + rb][lane] = acc[a][rb];
    }
    __syncthreads();
    if (wave > 0) return;
#pragma unroll
    for (int v = 0; v < kTailWaves - 1; ++v)
#pragma unroll
        for (int a = 0; a < NACC; ++a)
#pragma unroll
            for (int rb = 0; rb < RB; ++rb) {
                const f32x4_t p = part[v][a * RB + rb][lane];
#pragma unroll
                for (int j = 0; j < 4; ++j) acc[a][rb][j] = acc[a][rb][j] + p[j];
            }

    // Lane: column (feature) c0 + r16, rows 16 rb + 4 grp + j.
    const int64_t col = c0 + r16;
    if (SWIGLU) {
        const int64_t gr = wr0 + r16;  // gate weight row; up = gr + 32
        const float bg = HAS_BIAS ? __uint_as_float((uint32_t)bias[gr] << 16) : 0.0f;
        const float bu = HAS_BIAS ? __uint_as_float((uint32_t)bias[gr + 32] << 16) : 0.0f;
        uint16_t* yo = (uint16_t*)y;
#pragma unroll
        for (int rb = 0; rb < RB; ++rb)
#pragma unroll
            for (int j = 0; j < 4; j += 2) {
                uint32_t o0, o1;
                swiglu_bits2(acc[0][rb][j], acc[1][rb][j], acc[0][rb][j + 1], acc[1][rb][j + 1],
                             bg, bu, o0, o1);
                const int64_t r = 16 * rb + 4 * grp + j;
                if (r < R) yo[r * N + col] = (uint16_t)o0;
                if (r + 1 < R) yo[(r + 1) * N + col] = (uint16_t)o1;
            }
        return;
    }
    const float bv = HAS_BIAS ? __uint_as_float((uint32_t)bias[col] << 16) : 0.0f;
#pragma unroll
    for (int rb = 0; rb < RB; ++rb)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int64_t r = 16 * rb + 4 * grp + j;
            if (r >= R) continue;
            float v = acc[0][rb][j];
            if (HAS_BIAS) v = v + bv;
            const int64_t off = r * N + col;
            if (OUT_MODE == NCM_OUT_F32) {
                ((float*)y)[off] = HAS_RES ? residual[off] + v : v;
            } else {
                uint32_t bits = bf16_bits_rne(flush_subnormal(v));
                if (HAS_RES) bits = bf16_bits_rne(residual[off] + __uint_as_float(bits << 16));
                if (OUT_MODE == NCM_OUT_BF16_F32)
                    ((float*)y)[off] = __uint_as_float(bits << 16);
                else
                    ((uint16_t*)y)[off] = (uint16_t)bits;
            }
        }
}

template <int RB, bool SWIGLU, int OUT_MODE, bool HAS_BIAS, bool HAS_RES>
hipError_t launch_tail_t(const uint16_t* x, const uint16_t* w, const uint16_t* bias,
                         const float* residual, void* y, int64_t R, int64_t K, int64_t N,
                         hipStream_t st) {
    // Plain: N output columns; SwiGLU: N = features (weight rows 2 N).
    auto kern = linear_tail_kernel<RB, SWIGLU, OUT_MODE, HAS_BIAS, HAS_RES>;
    constexpr int lds = tail_lds_bytes<RB>();
    static const hipError_t attr = hipFuncSetAttribute(
        (const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, lds);
    if (attr != hipSuccess) return attr;
    hipLaunchKernelGGL(kern, dim3((unsigned)(N / 16)), dim3(64 * kTailWaves), lds, st, x, w,
                       bias, residual, y, R, K, N);
    return hipGetLastError();
}

template <int RB>
hipError_t launch_tail_rb(const uint16_t* x, const uint16_t* w, const uint16_t* bias,
                          const float* residual, void* y, int64_t R, int64_t K, int64_t N,
                          int out_mode, bool swiglu, hipStream_t st) {
    const bool hb = bias != nullptr, hr = residual != nullptr;
    if (swiglu)
        return hb ? launch_tail_t<RB, true, NCM_OUT_BF16, true, false>(x, w, bias, nullptr, y, R,
                                                                       K, N, st)
                  : launch_tail_t<RB, true, NCM_OUT_BF16, false, false>(x, w, bias, nullptr, y, R,
                                                                        K, N, st);
#define NCM_TAIL(MODE)                                                                         \
    (hb ? (hr ? launch_tail_t<RB, false, MODE, true, true>(x, w, bias, residual, y, R, K, N, st) \
              : launch_tail_t<RB, false, MODE, true, false>(x, w, bias, residual, y, R, K, N,    \
                                                            st))                               \
        : (hr ? launch_tail_t<RB, false, MODE, false, true>(x, w, bias, residual, y, R, K, N,    \
                                                            st)                                \
              : launch_tail_t<RB, false, MODE, false, false>(x, w, bias, residual, y, R, K, N,   \
                                                             st)))
    switch (out_mode) {
        case NCM_OUT_F32: return NCM_TAIL(NCM_OUT_F32);
        case NCM_OUT_BF16_F32: return NCM_TAIL(NCM_OUT_BF16_F32);
        default: return NCM_TAIL(NCM_OUT_BF16);
    }
#undef NCM_TAIL
}

}  // namespace

int64_t linear_tail_rows(int64_t M, int64_t N, int64_t K) {
    const int64_t r = M % 256;
    // K <= 2^22: every buffer offset the kernel forms, the out-of-range one
    // included, stays far below 2^32.
    if (r == 0 || r > kTailMaxRows || M < 256 || K % kTailKMultiple != 0 || N % 16 != 0 ||
        K > (int64_t)1 << 22)
        return 0;
    const int64_t m_main = M - r;
    if (linear_tile_config(M, N, K, -1) != 0 || linear_tile_config(m_main, N, K, -1) != 0)
        return 0;
    const int64_t cus = 256;
    const int64_t tiles_n = (N + 255) / 256;
    const int64_t rounds_main = ((m_main / 256) * tiles_n + cus - 1) / cus;
    const int64_t rounds_all = ((m_main / 256 + 1) * tiles_n + cus - 1) / cus;
    return rounds_all > rounds_main ? r : 0;
}

hipError_t launch_linear_tail(const uint16_t* x, const uint16_t* w, const uint16_t* bias,
                              const float* residual, void* y, int64_t R, int64_t K, int64_t N,
                              int out_mode, bool swiglu, hipStream_t st) {
    if (R <= 0 || R > kTailMaxRows || K % kTailKMultiple != 0 || N % 16 != 0 ||
        K > (int64_t)1 << 22)
        return hipErrorInvalidValue;
    if (R <= 16) return launch_tail_rb<1>(x, w, bias, residual, y, R, K, N, out_mode, swiglu, st);
    if (R <= 32) return launch_tail_rb<2>(x, w, bias, residual, y, R, K, N, out_mode, swiglu, st);
    return launch_tail_rb<4>(x, w, bias, residual, y, R, K, N, out_mode, swiglu, st);
}

}  // namespace ncm
