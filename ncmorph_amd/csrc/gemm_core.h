// bf16 MFMA main loop shared by the linear and the RVQ distance kernels.
//
// Computes acc += A_tile * B_tile^T where both operands are row-major with
// the reduction dimension contiguous ("NT"): A rows are the M dimension,
// B rows the N dimension. Tiles BM x BK and BN x BK are staged through two
// LDS stages from PF register sets (PF K tiles in flight from HBM/L2 while
// one feeds the MFMAs). Each 16-byte chunk c of LDS row r is stored at chunk
// slot c ^ ((r / 2) % (BK/8)) (BK = 64) or c ^ ((r / 4) % 4) (BK = 32): a
// 16-lane phase of a ds_read_b128 covers 16 consecutive rows at one K
// offset, and this gives those 16 rows 16 distinct 16-byte bank groups of
// the 64-bank LDS.
//
// Fragment layout of v_mfma_f32_32x32x16_bf16 (wave64):
//   A: lane l holds A[l % 32][8 (l / 32) .. 8 (l / 32) + 7]
//   B: lane l holds B[l % 32][8 (l / 32) .. 8 (l / 32) + 7]   (B = N x K rows)
//   D: lane l, element i holds D[8 (i / 4) + 4 (l / 32) + i % 4][l % 32]
#pragma once

#include "common.h"

namespace ncm {

// BM x BN x BK tile, WGM x WGN wavefronts, PF prefetch register sets,
// OCC target wavefronts per SIMD (register budget 512 / OCC), FDB: double
// buffer the MFMA fragments across k-steps.
// SCHED: 0 compiler order; 1, 2 the compiler's iglp_opt(0 / 1) DS-MFMA
// interleave; 3 an explicit interleave of one MFMA and one fragment read;
// 4 (with FDB) scheduling fences: all fragment reads of k-step kk + 1 are
// issued before the MFMAs of k-step kk, which then hide their latency.
// DMA: global -> LDS directly (buffer_load ... lds), no staging registers
// and no ds_write instructions; this path uses PF == 1 and waits for its own
// loads (vmcnt) explicitly at each barrier.
template <int BM_, int BN_, int BK_, int WGM_, int WGN_, int PF_ = 1, int OCC_ = 1,
          bool FDB_ = false, int SCHED_ = 0, bool DMA_ = false>
struct GemmShape {
    static constexpr int BM = BM_, BN = BN_, BK = BK_, WGM = WGM_, WGN = WGN_;
    static constexpr int PF = PF_, OCC = OCC_;
    static constexpr bool FDB = FDB_;
    static constexpr int SCHED = SCHED_;
    static constexpr bool DMA = DMA_;
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
    // Rows sharing a swizzle pattern: 2 for 128-byte rows, 4 for 64-byte rows.
    static constexpr int SWZ_SHIFT = BK == 64 ? 1 : 2;
    static_assert(WM % 32 == 0 && WN % 32 == 0, "wave tile must be 32-aligned");
    static_assert(BK == 32 || BK == 64, "BK must be 32 or 64");
    static_assert(NT % CH == 0 && BM % RPP == 0 && BN % RPP == 0, "loader shape");
    static_assert(RPP % (CH << SWZ_SHIFT) == 0, "swizzle must not depend on the pass");
    static_assert(PF == 1 || PF == 2, "one or two prefetch sets");
    static_assert(!DMA || PF == 1, "direct-to-LDS loads use one stage in flight");
    // Direct-to-LDS: one wave instruction fills 1 KB = RPI rows.
    static constexpr int NW = WGM * WGN;
    static constexpr int RPI = 1024 / (BK * 2);
    static constexpr int A_DMA = BM / (NW * RPI);
    static constexpr int B_DMA = BN / (NW * RPI);
    static_assert(!DMA || (BM % (NW * RPI) == 0 && BN % (NW * RPI) == 0), "DMA loader shape");
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

    // Loader: thread t moves 16-byte chunk (t % CH) of rows t / CH + p * RPP.
    // Global offsets differ per pass by a uniform stride, added to the VGPR
    // offset (the buffer range check covers the VGPR and instruction offsets,
    // not the scalar one); LDS offsets by a constant (instruction offset):
    // the swizzle term is the same for every pass.
    const int chunk = tid % S::CH;
    const int prow = tid / S::CH;
    const uint32_t a_goff = (uint32_t)(prow * lda * 2 + chunk * 16);
    const uint32_t b_goff = (uint32_t)(prow * ldb * 2 + chunk * 16);
    const uint32_t a_pstride = (uint32_t)(S::RPP * lda * 2);
    const uint32_t b_pstride = (uint32_t)(S::RPP * ldb * 2);
    const uint32_t soff =
        (uint32_t)((prow * S::CH + (chunk ^ ((prow >> S::SWZ_SHIFT) & (S::CH - 1)))) * 16);

    u32x4_t ra[S::PF][S::A_PASS], rb[S::PF][S::B_PASS];
    auto gload = [&](int set, int64_t k0) {
        const bool valid = (k0 + chunk * 8) < K;
        const uint32_t kb = (uint32_t)(k0 * 2);
        const uint32_t va = valid ? a_goff + kb : kOobOffset;
        const uint32_t vb = valid ? b_goff + kb : kOobOffset;
#pragma unroll
        for (int p = 0; p < S::A_PASS; ++p)
            ra[set][p] = __builtin_amdgcn_raw_buffer_load_b128(rsa, va + p * a_pstride, 0, 0);
#pragma unroll
        for (int p = 0; p < S::B_PASS; ++p)
            rb[set][p] = __builtin_amdgcn_raw_buffer_load_b128(rsb, vb + p * b_pstride, 0, 0);
    };
    auto sstore = [&](int set, int stage) {
        char* base = lds + stage * S::LDS_STAGE + soff;
#pragma unroll
        for (int p = 0; p < S::A_PASS; ++p)
            *(u32x4_t*)(base + p * S::RPP * S::CH * 16) = ra[set][p];
#pragma unroll
        for (int p = 0; p < S::B_PASS; ++p)
            *(u32x4_t*)(base + S::LDS_A + p * S::RPP * S::CH * 16) = rb[set][p];
    };

    // Fragment rows are wave_base + lane % 32 with wave_base a multiple of 32,
    // so their swizzle term is ((lane % 32) >> SWZ_SHIFT) % CH.
    const int frow = lane & 31;
    const int khalf = lane >> 5;
    const int swz = (frow >> S::SWZ_SHIFT) & (S::CH - 1);
    const uint32_t a_frag0 = (uint32_t)((wm * S::WM + frow) * S::CH * 16);
    const uint32_t b_frag0 = (uint32_t)(S::LDS_A + (wn * S::WN + frow) * S::CH * 16);

    constexpr int NFS = S::FDB ? 2 : 1;
    bf16x8_t af[NFS][S::MB], bfr[NFS][S::NB];
    auto fload = [&](int fs, const char* base, int kk) {
        const uint32_t cofs = (uint32_t)((((kk * 2 + khalf) ^ swz)) * 16);
#pragma unroll
        for (int mb = 0; mb < S::MB; ++mb)
            af[fs][mb] = *(const bf16x8_t*)(base + a_frag0 + mb * 32 * S::CH * 16 + cofs);
#pragma unroll
        for (int nb = 0; nb < S::NB; ++nb)
            bfr[fs][nb] = *(const bf16x8_t*)(base + b_frag0 + nb * 32 * S::CH * 16 + cofs);
    };
    auto mfmas = [&](int fs) {
#pragma unroll
        for (int mb = 0; mb < S::MB; ++mb)
#pragma unroll
            for (int nb = 0; nb < S::NB; ++nb)
                acc.v[mb][nb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
                    af[fs][mb], bfr[fs][nb], acc.v[mb][nb], 0, 0, 0);
    };
    // One LDS stage; with PF == 2 the other register set is written to the
    // other stage half-way through.
    auto compute = [&](int stage, int store_set, bool do_store) {
        const char* base = lds + stage * S::LDS_STAGE;
        if (S::FDB) fload(0, base, 0);
#pragma unroll
        for (int kk = 0; kk < S::KSTEPS; ++kk) {
            const int fs = S::FDB ? (kk & 1) : 0;
            if (S::FDB) {
                if (kk + 1 < S::KSTEPS) fload(fs ^ 1, base, kk + 1);
            } else {
                fload(0, base, kk);
            }
            if (S::SCHED == 4) __builtin_amdgcn_sched_barrier(0);
            mfmas(fs);
            if (S::SCHED == 4) __builtin_amdgcn_sched_barrier(0);
            if (S::PF == 2 && kk == S::KSTEPS / 2 - 1 && do_store) sstore(store_set, stage ^ 1);
            if (S::SCHED == 1) __builtin_amdgcn_iglp_opt(0);
            if (S::SCHED == 2) __builtin_amdgcn_iglp_opt(1);
            if (S::SCHED == 3 && S::FDB && kk + 1 < S::KSTEPS) {
                // MFMA, fragment read, MFMA, fragment read, ..., then the rest.
#pragma unroll
                for (int i = 0; i < S::MB + S::NB; ++i) {
                    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                    __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
                }
                __builtin_amdgcn_sched_group_barrier(0x008, S::MB * S::NB - (S::MB + S::NB), 0);
            }
        }
    };

    const int KT = (int)((K + S::BK - 1) / S::BK);
    if (S::DMA) {
        // Wave w, pass p fills LDS rows (p * NW + w) * RPI + lane / CH, slot
        // lane % CH, with the global chunk that the swizzle puts in that slot.
        const int drow0 = wave * S::RPI + lane / S::CH;
        const int dslot = lane % S::CH;
        auto dma = [&](int stage, int64_t k0) {
            char* sbase = lds + stage * S::LDS_STAGE;
            const uint32_t kb = (uint32_t)(k0 * 2);
#pragma unroll
            for (int p = 0; p < S::A_DMA + S::B_DMA; ++p) {
                const bool is_a = p < S::A_DMA;
                const int pp = is_a ? p : p - S::A_DMA;
                const int row = pp * S::NW * S::RPI + drow0;
                const int ch = dslot ^ ((row >> S::SWZ_SHIFT) & (S::CH - 1));
                const bool valid = (k0 + ch * 8) < K;
                const uint32_t off = (uint32_t)(row * (is_a ? lda : ldb) * 2 + ch * 16) + kb;
                char* dst = sbase + (is_a ? 0 : S::LDS_A) + (pp * S::NW + wave) * 1024;
                __builtin_amdgcn_raw_ptr_buffer_load_lds(
                    is_a ? rsa : rsb, (__attribute__((address_space(3))) void*)dst, 16,
                    valid ? off : kOobOffset, 0, 0, 0);
            }
        };
        // vmcnt(0) & lgkmcnt(0): this wave's LDS loads have landed and its
        // fragment reads are done, then the workgroup barrier.
        auto dma_barrier = [&]() {
            asm volatile("" ::: "memory");
            __builtin_amdgcn_s_waitcnt(0x0070);
            __builtin_amdgcn_s_barrier();
            asm volatile("" ::: "memory");
        };
        dma(0, 0);
        dma_barrier();
        for (int kt = 0; kt < KT; ++kt) {
            if (kt + 1 < KT) dma((kt + 1) & 1, (int64_t)(kt + 1) * S::BK);
            compute(kt & 1, 0, false);
            dma_barrier();
        }
        return;
    }
    if (S::PF == 1) {
        gload(0, 0);
        sstore(0, 0);
        lds_barrier();
        for (int kt = 0; kt < KT; ++kt) {
            if (kt + 1 < KT) gload(0, (int64_t)(kt + 1) * S::BK);
            compute(kt & 1, 0, false);
            if (kt + 1 < KT) sstore(0, (kt + 1) & 1);
            lds_barrier();
        }
    } else {
        gload(0, 0);
        if (KT > 1) gload(S::PF - 1, S::BK);
        sstore(0, 0);
        lds_barrier();
        int kt = 0;
        for (; kt + 1 < KT; kt += 2) {
            // Tile kt is in stage 0, tile kt + 1 in flight in set 1.
            if (kt + 2 < KT) gload(0, (int64_t)(kt + 2) * S::BK);
            compute(0, S::PF - 1, true);
            lds_barrier();
            // Tile kt + 1 is in stage 1, tile kt + 2 in flight in set 0.
            if (kt + 3 < KT) gload(S::PF - 1, (int64_t)(kt + 3) * S::BK);
            compute(1, 0, kt + 2 < KT);
            lds_barrier();
        }
        if (kt < KT) compute(0, 0, false);
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
