// The bf16 linear with epilogues that pair two 32-column MFMA tiles of one
// wave, fusing the elementwise op that follows the projection in the
// decoder (bf16 mode; the projection's own output is rounded to bf16 first,
// exactly as the unfused path writes it):
//   SwiGLU: weight rows are interleaved in groups of 32 (rows 64g .. 64g+31
//     are gate rows 32g .. 32g+31, rows 64g+32 .. 64g+63 the matching up
//     rows), so tiles 2p and 2p+1 of a wave hold gate and up of the same 32
//     features; the epilogue writes round(silu_bf16(gate) * up)
//     (src/decoder.zig:208-211) to y [M, N / 2].
//   RoPE (head_dim 64): tiles 2p and 2p+1 are the two halves of one head;
//     columns below rot_cols (the q and k heads) are rotated as rotate_head
//     does in bf16 mode (packages/kernels/root.zig:615-634) with table row
//     (row % seq_len), the rest (v) written as projected; y [M, N].
// Both write bf16 bits only.
#include "gemm_core.h"
#include "linear.h"

namespace ncm {

namespace {

constexpr int kEpiSwiGLU = 1;
constexpr int kEpiRope = 2;

struct PairArgs {
    const float* cosine;  // RoPE tables [seq_len, 64]
    const float* sine;
    int64_t seq_len;
    int64_t rot_cols;  // columns [0, rot_cols) are rotated
};

// The projections' output value of one accumulator is bf16(flush(acc +
// bias)), computed two values at a time with bf16x2_bits_rne (SwiGLU:
// swiglu_bits2 in common.h).

}  // namespace

template <class S, int EPI, bool HAS_BIAS>
__global__ __launch_bounds__(S::NT)
__attribute__((amdgpu_waves_per_eu(S::OCC, S::OCC))) void linear_pair_kernel(
    const void* __restrict__ x, const void* __restrict__ w, const uint16_t* __restrict__ bias,
    uint16_t* __restrict__ y, int64_t M, int64_t K, int64_t N, int tiles_n, int group_m,
    PairArgs pa) {
    static_assert(S::NB % 2 == 0 && S::WN % 64 == 0, "pairs of 32-column tiles per wave");
    extern __shared__ __attribute__((aligned(16))) char lds[];

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
    gemm_mainloop<S>((const char*)x + m0 * K * S::ESZ, K, operand_bytes(M, m0, K, S::ESZ),
                     (const char*)w + n0 * K * S::ESZ, K, operand_bytes(N, n0, K, S::ESZ), K, lds,
                     acc);

    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    if (wave >= S::NWG) return;
    const int wm = wave % S::WGM;
    const int wn = wave / S::WGM;
    const int c = lane & 31;
    const int64_t ld = EPI == kEpiSwiGLU ? N / 2 : N;

#pragma unroll
    for (int p = 0; p < S::NB / 2; ++p) {
        const int64_t col_a = n0 + wn * S::WN + 64 * p + c;  // first tile's column
        // N % 64 == 0: the pair is wholly in or out (wave-uniform).
        const bool in_range = col_a < N;
        float ba = 0.0f, bb = 0.0f;
        if (HAS_BIAS && in_range) {
            ba = __uint_as_float((uint32_t)bias[col_a] << 16);
            bb = __uint_as_float((uint32_t)bias[col_a + 32] << 16);
        }
        const bool rotate = EPI == kEpiRope && col_a < pa.rot_cols;
#pragma unroll
        for (int mb = 0; mb < S::MB; ++mb) {
            if (!in_range) break;
            // Per group of 4 rows: the projection's bits, a quad transpose
            // (each lane then holds 4 consecutive columns of one row, so
            // stores are 8 bytes and each RoPE table half is one 16-byte
            // load), then the fused op. Rows past M (a partial last row
            // tile) are computed on table row 0 and not stored.
            const int q = lane & 3;
            const int hrow = 4 * (lane >> 5) + q;
            const int c4 = c & ~3;
            const int64_t ca = EPI == kEpiSwiGLU ? (n0 + wn * S::WN) / 2 + 32 * p + c4
                                                 : col_a - c + c4;
#pragma unroll
            for (int blk = 0; blk < 4; ++blk) {
                const int64_t m = m0 + wm * S::WM + mb * 32 + 8 * blk + hrow;
                if (EPI == kEpiSwiGLU) {
                    // Elementwise first (gate and up of a column sit in the
                    // same lane and element), then one transpose of the
                    // results.
                    float r[4];
#pragma unroll
                    for (int j = 0; j < 4; j += 2) {
                        uint32_t o0, o1;
                        swiglu_bits2(acc.v[mb][2 * p][4 * blk + j], acc.v[mb][2 * p + 1][4 * blk + j],
                                     acc.v[mb][2 * p][4 * blk + j + 1],
                                     acc.v[mb][2 * p + 1][4 * blk + j + 1], ba, bb, o0, o1);
                        r[j] = __uint_as_float(o0);
                        r[j + 1] = __uint_as_float(o1);
                    }
                    quad_transpose4(r, q);
                    if (m < M) {
                        u32x2_t o;
                        o[0] = __float_as_uint(r[0]) | (__float_as_uint(r[1]) << 16);
                        o[1] = __float_as_uint(r[2]) | (__float_as_uint(r[3]) << 16);
                        __builtin_nontemporal_store(o, (u32x2_t*)(y + m * ld + ca));
                    }
                    continue;
                }
                // The two tiles' projection bits, bf16(flush(acc + bias)), one
                // v_cvt_pk_bf16_f32 per pair.
                float va[4], vb[4];
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const uint32_t pr =
                        bf16x2_bits_rne(flush_subnormal(acc.v[mb][2 * p][4 * blk + j] + ba),
                                        flush_subnormal(acc.v[mb][2 * p + 1][4 * blk + j] + bb));
                    va[j] = __uint_as_float(pr & 0xFFFFu);
                    vb[j] = __uint_as_float(pr >> 16);
                }
                quad_transpose4(va, q);
                quad_transpose4(vb, q);
                uint32_t ra[4], rbits[4];
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    ra[j] = __float_as_uint(va[j]);
                    rbits[j] = __float_as_uint(vb[j]);
                }
                if (rotate) {
                    const int64_t t = (m < M ? m : 0) % pa.seq_len;
                    const f32x4_t cf = *(const f32x4_t*)(pa.cosine + t * 64 + c4);
                    const f32x4_t cs = *(const f32x4_t*)(pa.cosine + t * 64 + 32 + c4);
                    const f32x4_t sf = *(const f32x4_t*)(pa.sine + t * 64 + c4);
                    const f32x4_t ss = *(const f32x4_t*)(pa.sine + t * 64 + 32 + c4);
                    // Per column: left = rb(first rb(cos)), right =
                    // rb(-second rb(sin)), right2 = rb(first rb(sin2)),
                    // left2 = rb(second rb(cos2)), then round(left + right)
                    // and round(left2 + right2); each rounding done for two
                    // columns at once (bf16x2_bits_rne, the bits of rb).
                    auto lo = [](uint32_t pr) { return __uint_as_float(pr << 16); };
                    auto hi = [](uint32_t pr) { return __uint_as_float(pr & 0xFFFF0000u); };
#pragma unroll
                    for (int j = 0; j < 4; j += 2) {
                        const float f0 = __uint_as_float(ra[j] << 16);
                        const float f1 = __uint_as_float(ra[j + 1] << 16);
                        const float s0 = __uint_as_float(rbits[j] << 16);
                        const float s1 = __uint_as_float(rbits[j + 1] << 16);
                        // Intermediates without the NaN rule (a NaN stays a
                        // NaN through products and sums; the final rounding
                        // maps it to 0x7FC0).
                        const uint32_t tc = bf16x2_rne(cf[j], cf[j + 1]);
                        const uint32_t ts = bf16x2_rne(sf[j], sf[j + 1]);
                        const uint32_t ts2 = bf16x2_rne(ss[j], ss[j + 1]);
                        const uint32_t tc2 = bf16x2_rne(cs[j], cs[j + 1]);
                        const uint32_t left = bf16x2_rne(f0 * lo(tc), f1 * hi(tc));
                        const uint32_t right = bf16x2_rne(-s0 * lo(ts), -s1 * hi(ts));
                        const uint32_t right2 = bf16x2_rne(f0 * lo(ts2), f1 * hi(ts2));
                        const uint32_t left2 = bf16x2_rne(s0 * lo(tc2), s1 * hi(tc2));
                        const uint32_t o1 = bf16x2_bits_rne(lo(left) + lo(right),
                                                            hi(left) + hi(right));
                        const uint32_t o2 = bf16x2_bits_rne(lo(left2) + lo(right2),
                                                            hi(left2) + hi(right2));
                        ra[j] = o1 & 0xFFFFu;
                        ra[j + 1] = o1 >> 16;
                        rbits[j] = o2 & 0xFFFFu;
                        rbits[j + 1] = o2 >> 16;
                    }
                }
                if (m < M) {
                    u32x2_t o;
                    o[0] = ra[0] | (ra[1] << 16);
                    o[1] = ra[2] | (ra[3] << 16);
                    __builtin_nontemporal_store(o, (u32x2_t*)(y + m * ld + ca));
                    if (EPI == kEpiRope) {
                        o[0] = rbits[0] | (rbits[1] << 16);
                        o[1] = rbits[2] | (rbits[3] << 16);
                        __builtin_nontemporal_store(o, (u32x2_t*)(y + m * ld + ca + 32));
                    }
                }
            }
        }
    }
}

template <class S, int EPI, bool HAS_BIAS>
static hipError_t launch_pair_t(const uint16_t* x, const uint16_t* w, const uint16_t* bias,
                                uint16_t* y, int64_t M, int64_t K, int64_t N, PairArgs pa,
                                hipStream_t stream) {
    auto kern = linear_pair_kernel<S, EPI, HAS_BIAS>;
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
                       bias, y, M, K, N, tiles_n, group_m, pa);
    return hipGetLastError();
}

template <int EPI>
static hipError_t launch_pair(const uint16_t* x, const uint16_t* w, const uint16_t* bias,
                              uint16_t* y, int64_t M, int64_t K, int64_t N, PairArgs pa,
                              hipStream_t st) {
    using L0 = GemmShape<256, 256, 64, 4, 2, 2, 8, true, 2, false, 1, -1, -1, true>;
    using L1 = GemmShape<128, 128, 64, 4, 2, 2, 8, true, 4, false, 1, -1, -1, true>;
    using L2 = GemmShape<128, 128, 64, 2, 2, 2, 4, true>;
    using L5 = GemmShape<256, 128, 64, 4, 2, 2, 8, true, 3, false, 1, -1, -1, true>;
    const bool hb = bias != nullptr;
    switch (linear_tile_config(M, N, K, -1)) {
        case 0:
            return hb ? launch_pair_t<L0, EPI, true>(x, w, bias, y, M, K, N, pa, st)
                      : launch_pair_t<L0, EPI, false>(x, w, bias, y, M, K, N, pa, st);
        case 1:
            return hb ? launch_pair_t<L1, EPI, true>(x, w, bias, y, M, K, N, pa, st)
                      : launch_pair_t<L1, EPI, false>(x, w, bias, y, M, K, N, pa, st);
        case 5:
            return hb ? launch_pair_t<L5, EPI, true>(x, w, bias, y, M, K, N, pa, st)
                      : launch_pair_t<L5, EPI, false>(x, w, bias, y, M, K, N, pa, st);
        default:
            return hb ? launch_pair_t<L2, EPI, true>(x, w, bias, y, M, K, N, pa, st)
                      : launch_pair_t<L2, EPI, false>(x, w, bias, y, M, K, N, pa, st);
    }
}

hipError_t launch_linear_swiglu(const uint16_t* x, const uint16_t* w, const uint16_t* bias,
                                uint16_t* y, int64_t M, int64_t K, int64_t N2,
                                hipStream_t stream) {
    if (N2 % 64) return hipErrorInvalidValue;
    const int64_t r = linear_tail_rows(M, N2, K);
    if (r > 0) {
        const int64_t mm = M - r;
        hipError_t e = launch_pair<kEpiSwiGLU>(x, w, bias, y, mm, K, N2,
                                               PairArgs{nullptr, nullptr, 1, 0}, stream);
        if (e != hipSuccess) return e;
        return launch_linear_tail(x + mm * K, w, bias, nullptr, y + mm * (N2 / 2), r, K, N2 / 2,
                                  NCM_OUT_BF16, true, stream);
    }
    return launch_pair<kEpiSwiGLU>(x, w, bias, y, M, K, N2, PairArgs{nullptr, nullptr, 1, 0},
                                   stream);
}

hipError_t launch_linear_rope64(const uint16_t* x, const uint16_t* w, const uint16_t* bias,
                                uint16_t* y, int64_t M, int64_t K, int64_t N, int64_t rot_cols,
                                int64_t seq_len, const float* cosine, const float* sine,
                                hipStream_t stream) {
    if (N % 64 || rot_cols % 64 || seq_len <= 0) return hipErrorInvalidValue;
    return launch_pair<kEpiRope>(x, w, bias, y, M, K, N,
                                 PairArgs{cosine, sine, seq_len, rot_cols}, stream);
}

}  // namespace ncm
