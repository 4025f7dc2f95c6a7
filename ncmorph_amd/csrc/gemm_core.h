// bf16 MFMA main loop shared by the linear and the RVQ distance kernels.
//
// Computes acc += A_tile * B_tile^T where both operands are row-major with
// the reduction dimension contiguous ("NT"): A rows are the M dimension,
// B rows the N dimension. Tiles BM x BK and BN x BK are staged through LDS
// (two stages, register prefetch of the next K tile while the current one
// feeds the MFMAs). Each 16-byte chunk c of LDS row r is stored at chunk
// slot c ^ (r % (BK/8)), so the 32 rows a v_mfma_f32_32x32x16_bf16 operand
// reads at one K offset hit distinct banks.
//
// Fragment layout of v_mfma_f32_32x32x16_bf16 (wave64):
//   A: lane l holds A[l % 32][8 (l / 32) .. 8 (l / 32) + 7]
//   B: lane l holds B[l % 32][8 (l / 32) .. 8 (l / 32) + 7]   (B = N x K rows)
//   D: lane l, element i holds D[8 (i / 4) + 4 (l / 32) + i % 4][l % 32]
#pragma once

#include "common.h"

namespace ncm {

template <int BM_, int BN_, int BK_, int WGM_, int WGN_>
struct GemmShape {
    static constexpr int BM = BM_, BN = BN_, BK = BK_, WGM = WGM_, WGN = WGN_;
    static constexpr int NT = kWave * WGM * WGN;
    static constexpr int WM = BM / WGM, WN = BN / WGN;
    static constexpr int MB = WM / 32, NB = WN / 32;
    static constexpr int CH = BK / 8;
    static constexpr int KSTEPS = BK / 16;
    static constexpr int RPP = NT / CH;
    static constexpr int A_PASS = BM / RPP;
    static constexpr int B_PASS = BN / RPP;
    static constexpr int LDS_A = BM * BK * 2;
    static constexpr int LDS_B = BN * BK * 2;
    static constexpr int LDS_STAGE = LDS_A + LDS_B;
    static constexpr int LDS_BYTES = 2 * LDS_STAGE;
    static_assert(WM % 32 == 0 && WN % 32 == 0, "wave tile must be 32-aligned");
    static_assert(BK % 16 == 0 && (CH & (CH - 1)) == 0, "BK must be 16 * 2^k");
    static_assert(NT % CH == 0 && BM % RPP == 0 && BN % RPP == 0, "loader shape");
    static_assert(LDS_BYTES <= 160 * 1024, "LDS budget of a gfx950 CU");
};

template <class S>
struct GemmAcc {
    f32x16_t v[S::MB][S::NB];
    __device__ __forceinline__ void zero() {
#pragma unroll
        for (int i = 0; i < S::MB; ++i)
#pragma unroll
            for (int j = 0; j < S::NB; ++j)
#pragma unroll
                for (int e = 0; e < 16; ++e) v[i][j][e] = 0.0f;
    }
};

// A points at the tile's first row; a_bytes is how many bytes from A are
// readable (rows past it load as zero). Same for B. K % 8 == 0; K-chunks at
// or past K load as zero.
template <class S>
__device__ __forceinline__ void gemm_mainloop(const uint16_t* A, int64_t lda, uint32_t a_bytes,
                                              const uint16_t* B, int64_t ldb, uint32_t b_bytes,
                                              int64_t K, char* lds, GemmAcc<S>& acc) {
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int wm = wave % S::WGM;
    const int wn = wave / S::WGM;

    const __amdgpu_buffer_rsrc_t rsa = make_rsrc(A, a_bytes);
    const __amdgpu_buffer_rsrc_t rsb = make_rsrc(B, b_bytes);

    const int chunk = tid % S::CH;
    const int prow = tid / S::CH;
    uint32_t a_goff[S::A_PASS], b_goff[S::B_PASS];
    uint32_t a_soff[S::A_PASS], b_soff[S::B_PASS];
#pragma unroll
    for (int p = 0; p < S::A_PASS; ++p) {
        const int r = prow + p * S::RPP;
        a_goff[p] = (uint32_t)(r * lda * 2 + chunk * 16);
        a_soff[p] = (uint32_t)((r * S::CH + (chunk ^ (r & (S::CH - 1)))) * 16);
    }
#pragma unroll
    for (int p = 0; p < S::B_PASS; ++p) {
        const int r = prow + p * S::RPP;
        b_goff[p] = (uint32_t)(r * ldb * 2 + chunk * 16);
        b_soff[p] = (uint32_t)(S::LDS_A + (r * S::CH + (chunk ^ (r & (S::CH - 1)))) * 16);
    }

    u32x4_t ra[S::A_PASS], rb[S::B_PASS];
    auto gload = [&](int64_t k0) {
        const bool valid = (k0 + chunk * 8) < K;
        const uint32_t kb = (uint32_t)(k0 * 2);
#pragma unroll
        for (int p = 0; p < S::A_PASS; ++p)
            ra[p] = buffer_load_b128(rsa, valid ? a_goff[p] + kb : kOobOffset);
#pragma unroll
        for (int p = 0; p < S::B_PASS; ++p)
            rb[p] = buffer_load_b128(rsb, valid ? b_goff[p] + kb : kOobOffset);
    };
    auto sstore = [&](int stage) {
        char* base = lds + stage * S::LDS_STAGE;
#pragma unroll
        for (int p = 0; p < S::A_PASS; ++p) *(u32x4_t*)(base + a_soff[p]) = ra[p];
#pragma unroll
        for (int p = 0; p < S::B_PASS; ++p) *(u32x4_t*)(base + b_soff[p]) = rb[p];
    };

    // Fragment rows: (row & (CH - 1)) == (lane & (CH - 1)) because the
    // other row terms are multiples of 32.
    const int frow = lane & 31;
    const int khalf = lane >> 5;
    const int swz = lane & (S::CH - 1);
    const uint32_t a_frag0 = (uint32_t)((wm * S::WM + frow) * S::CH * 16);
    const uint32_t b_frag0 = (uint32_t)(S::LDS_A + (wn * S::WN + frow) * S::CH * 16);

    const int KT = (int)((K + S::BK - 1) / S::BK);
    gload(0);
    sstore(0);
    __syncthreads();
    for (int kt = 0; kt < KT; ++kt) {
        if (kt + 1 < KT) gload((int64_t)(kt + 1) * S::BK);
        const char* base = lds + (kt & 1) * S::LDS_STAGE;
#pragma unroll
        for (int kk = 0; kk < S::KSTEPS; ++kk) {
            const uint32_t cofs = (uint32_t)((((kk * 2 + khalf) ^ swz)) * 16);
            bf16x8_t af[S::MB], bfr[S::NB];
#pragma unroll
            for (int mb = 0; mb < S::MB; ++mb)
                af[mb] = *(const bf16x8_t*)(base + a_frag0 + mb * 32 * S::CH * 16 + cofs);
#pragma unroll
            for (int nb = 0; nb < S::NB; ++nb)
                bfr[nb] = *(const bf16x8_t*)(base + b_frag0 + nb * 32 * S::CH * 16 + cofs);
#pragma unroll
            for (int mb = 0; mb < S::MB; ++mb)
#pragma unroll
                for (int nb = 0; nb < S::NB; ++nb)
                    acc.v[mb][nb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
                        af[mb], bfr[nb], acc.v[mb][nb], 0, 0, 0);
        }
        if (kt + 1 < KT) sstore((kt + 1) & 1);
        __syncthreads();
    }
}

// Bytes of a row-major operand readable from row `row0` of `rows`, capped so
// that every offset the loader forms stays below kOobOffset.
__host__ __device__ inline uint32_t operand_bytes(int64_t rows, int64_t row0, int64_t ld) {
    int64_t left = rows - row0;
    if (left <= 0) return 0;
    int64_t b = left * ld * 2;
    return b >= (int64_t)kOobOffset ? kOobOffset - 16u : (uint32_t)b;
}

}  // namespace ncm
