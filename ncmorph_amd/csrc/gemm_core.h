// MFMA main loop shared by the linear kernels (bf16 and fp32 operands) and
// the RVQ distance kernel.
//
// Computes acc += A_tile * B_tile^T where both operands are row-major with
// the reduction dimension contiguous ("NT"): A rows are the M dimension,
// B rows the N dimension. A K tile is RB = BK * element-size bytes per row
// (64, 128 or 256). Each 16-byte chunk c of LDS row r is stored at chunk
// slot c ^ (r % 16) (RB = 256), c ^ ((r / 2) % 8) (RB = 128) or
// c ^ ((r / 4) % 4) (RB = 64): a 16-lane phase of a ds_read_b128 covers 16
// consecutive rows at one K offset, and this gives those 16 rows 16 distinct
// 16-byte bank groups of the 64-bank LDS.
//
// A k-step consumes two 16-byte chunks of every row: lanes 0-31 read chunk
// 2 kk, lanes 32-63 chunk 2 kk + 1, of row (lane % 32) of a 32-row block.
//   bf16: one v_mfma_f32_32x32x16_bf16; lane l supplies
//         A[l % 32][8 (l / 32) .. 8 (l / 32) + 7] of the k-step (B alike).
//   fp32: four v_mfma_f32_32x32x2_f32; MFMA j takes element j of each
//         lane's chunk, i.e. the pair of K indices (j, 4 + j) of the k-step.
//         A and B use the same pairing, so the four MFMAs sum every product
//         of the k-step exactly once.
//   D (both): lane l, element i holds D[8 (i / 4) + 4 (l / 32) + i % 4][l % 32].
#pragma once

#include <type_traits>

#include "common.h"

namespace ncm {

// BM x BN x BK tile (BK in elements), WGM x WGN wavefronts, OCC target
// wavefronts per SIMD (register budget 512 / OCC).
// SCHED:
//   0  compiler order, one fragment set (register-staged loads only);
//   4  fragment double buffering with scheduling fences: the fragment reads
//      of k-step kk + 1 are issued before the MFMAs of k-step kk;
//   5  (DMA) as 4, and the K-tile barrier sits in the middle of the last
//      k-step's MFMAs, followed by the next stage's first fragment reads,
//      so the second half of those MFMAs covers the barrier and the LDS
//      latency;
//   6  (DMA, NST >= 3) ping-pong: the wavefronts form two groups (one
//      wavefront of each per SIMD) that run half a K tile apart. Between
//      two barriers one group issues all MFMAs of a tile from registers
//      while the other reads the next tile's fragments from LDS and issues
//      its share of the direct-to-LDS loads;
//   7  (DMA, KG = 2, NST even >= 4) K groups: two groups of WGM x WGN
//      wavefronts (one wavefront of each per SIMD) each accumulate the whole
//      output tile over alternate K tiles (group g takes tiles 2i + g) from
//      one shared pipeline, NST / 2 - 1 tile pairs ahead; at the end group 1
//      hands its accumulators to group 0 through LDS and group 0 holds
//      acc(group 0) + acc(group 1).
//   8  (DMA) SCHED 5's stage rotation and barrier, with each tile's loads
//      spread over its first DSPREAD k-steps and, inside a k-step, the
//      loads and the next k-step's fragment reads placed one by one between
//      the MFMAs (scheduling-group barriers): the matrix core keeps working
//      while they issue instead of waiting for a block of them.
// DMA: global -> LDS directly (buffer_load ... lds), no staging registers
// and no ds_write instructions; this path waits for its own loads (vmcnt)
// explicitly at each barrier. Without DMA, one K tile is staged through
// registers while the previous one feeds the MFMAs.
// NST: LDS stages of the DMA path; K tiles up to NST - 1 ahead are in flight.
// F32: fp32 operands (else bf16). KG: K groups (SCHED 7).
// MF16: (bf16, SCHED 8) v_mfma_f32_16x16x32_bf16 on 16-row fragments
// instead of v_mfma_f32_32x32x16_bf16; the main loop converts the
// accumulators to the 32x32x16 layout at its end, so epilogues are the same.
template <int BM_, int BN_, int BK_, int WGM_, int WGN_, int OCC_, int SCHED_, bool DMA_,
          int NST_ = 2, bool F32_ = false, int KG_ = 1, int BS_ = -1, int DSP_ = -1,
          bool MF16_ = false>
struct GemmShape {
    static constexpr int BM = BM_, BN = BN_, BK = BK_, WGM = WGM_, WGN = WGN_;
    static constexpr int OCC = OCC_, SCHED = SCHED_, NST = NST_, KG = KG_;
    static constexpr bool DMA = DMA_, F32 = F32_;
    static constexpr bool FDB = SCHED >= 4;
    static constexpr int ESZ = F32 ? 4 : 2;
    static constexpr int EPC = 16 / ESZ;  // elements per 16-byte chunk
    static constexpr int RB = BK * ESZ;   // bytes per tile row
    static constexpr int NT = kWave * WGM * WGN * KG;
    static constexpr int NW = WGM * WGN * KG;
    static constexpr int NWG = WGM * WGN;  // wavefronts per K group
    static constexpr int WM = BM / WGM, WN = BN / WGN;
    static constexpr int MB = WM / 32, NB = WN / 32;
    static constexpr bool MF16 = MF16_;
    // Fragments (A, B) and MFMAs of one k-step; a k-step is 16 (32x32x16) or
    // 32 (16x16x32) elements of K.
    static constexpr int FM = MF16 ? 2 * MB : MB, FN = MF16 ? 2 * NB : NB;
    static constexpr int NMFS = FM * FN;
    // SCHED 5 and 8: MFMAs of the last k-step issued before the K-tile barrier.
    static constexpr int BSPLIT = BS_ < 0 ? NMFS / 2 : BS_;
    static constexpr int CH = RB / 16;
    static constexpr int KSTEPS = MF16 ? CH / 4 : CH / 2;
    // SCHED 8: k-steps over which a tile's direct-to-LDS loads are spread.
    static constexpr int DSPREAD = DSP_ < 0 ? KSTEPS - 1 : DSP_;
    static constexpr int RPP = NT / CH;
    static constexpr int A_PASS = BM / RPP;
    static constexpr int B_PASS = BN / RPP;
    static constexpr int LDS_A = BM * RB;
    static constexpr int LDS_B = BN * RB;
    static constexpr int LDS_STAGE = LDS_A + LDS_B;
    static constexpr int LDS_BYTES = NST * LDS_STAGE;
    // Rows sharing a swizzle pattern: 1, 2 or 4 for 256-, 128- or 64-byte rows.
    static constexpr int SWZ_SHIFT = RB == 256 ? 0 : (RB == 128 ? 1 : 2);
    // Direct-to-LDS: one wave instruction fills 1 KB = RPI rows.
    static constexpr int RPI = 1024 / RB;
    static constexpr int A_DMA = BM / (NW * RPI);
    static constexpr int B_DMA = BN / (NW * RPI);
    static_assert(WM % 32 == 0 && WN % 32 == 0, "wave tile must be 32-aligned");
    static_assert(RB == 64 || RB == 128 || RB == 256, "a K tile row is 64, 128 or 256 bytes");
    static_assert(NT % CH == 0 && BM % RPP == 0 && BN % RPP == 0, "loader shape");
    static_assert(RPP % (CH << SWZ_SHIFT) == 0, "swizzle must not depend on the pass");
    static_assert(SCHED == 0 || SCHED == 4 || SCHED == 5 || SCHED == 6 || SCHED == 7 ||
                      SCHED == 8,
                  "schedule");
    static_assert((KG == 2) == (SCHED == 7), "K groups go with SCHED 7");
    static_assert(SCHED != 7 || (NST % 2 == 0 && NST >= 4), "SCHED 7 stages come in pairs");
    static_assert(DMA || SCHED <= 4, "SCHED 5, 6 and 7 need direct-to-LDS loads");
    static_assert(!MF16 || (SCHED == 8 && !F32 && CH % 4 == 0), "16x16x32: bf16, SCHED 8");
    static_assert(!DMA || SCHED >= 4, "direct-to-LDS loads need fragment double buffering");
    static_assert(!DMA || (BM % (NW * RPI) == 0 && BN % (NW * RPI) == 0), "DMA loader shape");
    static_assert(NST == 2 || SCHED >= 5, "more than two stages: SCHED 5, 6 or 7 only");
    static_assert(SCHED != 6 || (NST >= 3 && NW % 2 == 0), "ping-pong layout");
    static_assert((SCHED != 5 && SCHED != 8) || KSTEPS % 2 == 0,
                  "SCHED 5 and 8 split the last k-step pair");
    static_assert(SCHED != 8 || KSTEPS >= 2, "SCHED 8 spreads the loads over the first k-steps");
    static_assert(NST >= 2 && (NST - 2) * (A_DMA + B_DMA) <= 63, "vmcnt range");
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

// One k-step of one 32 x 32 accumulator block.
template <class S>
__device__ __forceinline__ void mfma_kstep(f32x16_t& c, const u32x4_t& a, const u32x4_t& b) {
    if constexpr (S::F32) {
#pragma unroll
        for (int j = 0; j < 4; ++j)
            c = __builtin_amdgcn_mfma_f32_32x32x2f32(__uint_as_float(a[j]), __uint_as_float(b[j]),
                                                     c, 0, 0, 0);
    } else {
        c = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                    __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
    }
}

// s_waitcnt immediate: vmcnt(vm) & lgkmcnt(0), expcnt unconstrained.
constexpr int waitcnt_vm_lgkm0(int vm) { return (vm & 0xF) | ((vm >> 4) << 14) | (0x7 << 4); }

// Wait for vmcnt(VM) and this wave's LDS operations, then the workgroup
// barrier; the empty asm statements keep the compiler from moving memory
// operations across it.
template <int VM>
__device__ __forceinline__ void wait_barrier() {
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt(waitcnt_vm_lgkm0(VM));
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

// A points at the tile's first row; a_bytes is how many bytes from A are
// readable (rows past it load as zero). Same for B. lda, ldb and K are in
// elements, K % (16 / element size) == 0; K-chunks at or past K load as
// zero.
template <class S>
__device__ __forceinline__ void gemm_mainloop(const void* A, int64_t lda, uint32_t a_bytes,
                                              const void* B, int64_t ldb, uint32_t b_bytes,
                                              int64_t K, char* lds, GemmAcc<S>& acc) {
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wl = wave % S::NWG;  // wavefront inside its K group
    const int wm = wl % S::WGM;
    const int wn = wl / S::WGM;

    const __amdgpu_buffer_rsrc_t rsa = make_rsrc(A, a_bytes);
    const __amdgpu_buffer_rsrc_t rsb = make_rsrc(B, b_bytes);

    // Fragment rows are wave_base + lane % FR (FR = 32, or 16 for 16x16x32)
    // with wave_base a multiple of FR, so their swizzle term is
    // ((lane % FR) >> SWZ_SHIFT) % CH; a k-step reads CPK chunks of each row,
    // lane / FR picking the chunk.
    constexpr int FR = S::MF16 ? 16 : 32;
    constexpr int CPK = S::MF16 ? 4 : 2;
    const int frow = lane & (FR - 1);
    const int khalf = lane / FR;
    const int swz = (frow >> S::SWZ_SHIFT) & (S::CH - 1);
    const uint32_t a_frag0 = (uint32_t)((wm * S::WM + frow) * S::RB);
    const uint32_t b_frag0 = (uint32_t)(S::LDS_A + (wn * S::WN + frow) * S::RB);

    constexpr int NFS = S::FDB ? 2 : 1;
    u32x4_t af[NFS][S::FM], bfr[NFS][S::FN];
    auto fload = [&](int fs, const char* base, int kk) {
        const uint32_t cofs = (uint32_t)((((kk * CPK + khalf) ^ swz)) * 16);
#pragma unroll
        for (int mb = 0; mb < S::FM; ++mb)
            af[fs][mb] = *(const u32x4_t*)(base + a_frag0 + mb * FR * S::RB + cofs);
#pragma unroll
        for (int nb = 0; nb < S::FN; ++nb)
            bfr[fs][nb] = *(const u32x4_t*)(base + b_frag0 + nb * FR * S::RB + cofs);
    };
    // Fragment j of k-step kk: A block j (j < FM) or B block j - FM.
    auto fload_one = [&](int fs, const char* base, int kk, int j) {
        const uint32_t cofs = (uint32_t)((((kk * CPK + khalf) ^ swz)) * 16);
        if (j < S::FM)
            af[fs][j] = *(const u32x4_t*)(base + a_frag0 + j * FR * S::RB + cofs);
        else
            bfr[fs][j - S::FM] =
                *(const u32x4_t*)(base + b_frag0 + (j - S::FM) * FR * S::RB + cofs);
    };
    // MFMAs lo .. hi - 1 of one k-step, in (A block, B block) row-major order.
    // 16x16x32: 16-row blocks (2 mb + sa, 2 nb + sb) accumulate into elements
    // 4 (2 sa + sb) .. + 3 of the 32x32 block (mb, nb) until the end of the
    // main loop converts them.
    auto mfma_range = [&](int fs, int lo, int hi) {
#pragma unroll
        for (int i = 0; i < S::NMFS; ++i) {
            if (i < lo || i >= hi) continue;
            const int ia = i / S::FN, ib = i % S::FN;
            if constexpr (S::MF16) {
                f32x16_t& c = acc.v[ia >> 1][ib >> 1];
                const int e0 = 4 * (2 * (ia & 1) + (ib & 1));
                f32x4_t d;
                d[0] = c[e0]; d[1] = c[e0 + 1]; d[2] = c[e0 + 2]; d[3] = c[e0 + 3];
                d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                    __builtin_bit_cast(bf16x8_t, af[fs][ia]),
                    __builtin_bit_cast(bf16x8_t, bfr[fs][ib]), d, 0, 0, 0);
                c[e0] = d[0]; c[e0 + 1] = d[1]; c[e0 + 2] = d[2]; c[e0 + 3] = d[3];
            } else {
                mfma_kstep<S>(acc.v[ia][ib], af[fs][ia], bfr[fs][ib]);
            }
        }
    };
    constexpr int NMF = S::NMFS;
    // All k-steps of one LDS stage (SCHED 0 and 4).
    auto compute = [&](int stage) {
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
            if (S::SCHED == 4 || S::SCHED == 7) __builtin_amdgcn_sched_barrier(0);
            mfma_range(fs, 0, NMF);
            if (S::SCHED == 4 || S::SCHED == 7) __builtin_amdgcn_sched_barrier(0);
        }
    };

    const int KT = (int)((K + S::BK - 1) / S::BK);

    if (!S::DMA) {
        // Register-staged loads: thread t moves 16-byte chunk (t % CH) of
        // rows t / CH + p * RPP. Global offsets differ per pass by a uniform
        // stride, added to the VGPR offset (the buffer range check covers
        // the VGPR and instruction offsets, not the scalar one); LDS offsets
        // by a constant: the swizzle term is the same for every pass.
        const int chunk = tid % S::CH;
        const int prow = tid / S::CH;
        const uint32_t a_goff = (uint32_t)(prow * lda * S::ESZ + chunk * 16);
        const uint32_t b_goff = (uint32_t)(prow * ldb * S::ESZ + chunk * 16);
        const uint32_t a_pstride = (uint32_t)(S::RPP * lda * S::ESZ);
        const uint32_t b_pstride = (uint32_t)(S::RPP * ldb * S::ESZ);
        const uint32_t soff =
            (uint32_t)(prow * S::RB + (chunk ^ ((prow >> S::SWZ_SHIFT) & (S::CH - 1))) * 16);
        u32x4_t ra[S::A_PASS], rb[S::B_PASS];
        auto gload = [&](int64_t k0) {
            const bool valid = (k0 + chunk * S::EPC) < K;
            const uint32_t kb = (uint32_t)(k0 * S::ESZ);
            const uint32_t va = valid ? a_goff + kb : kOobOffset;
            const uint32_t vb = valid ? b_goff + kb : kOobOffset;
#pragma unroll
            for (int p = 0; p < S::A_PASS; ++p)
                ra[p] = __builtin_amdgcn_raw_buffer_load_b128(rsa, va + p * a_pstride, 0, 0);
#pragma unroll
            for (int p = 0; p < S::B_PASS; ++p)
                rb[p] = __builtin_amdgcn_raw_buffer_load_b128(rsb, vb + p * b_pstride, 0, 0);
        };
        auto sstore = [&](int stage) {
            char* base = lds + stage * S::LDS_STAGE + soff;
#pragma unroll
            for (int p = 0; p < S::A_PASS; ++p) *(u32x4_t*)(base + p * S::RPP * S::RB) = ra[p];
#pragma unroll
            for (int p = 0; p < S::B_PASS; ++p)
                *(u32x4_t*)(base + S::LDS_A + p * S::RPP * S::RB) = rb[p];
        };
        gload(0);
        sstore(0);
        lds_barrier();
        for (int kt = 0; kt < KT; ++kt) {
            if (kt + 1 < KT) gload((int64_t)(kt + 1) * S::BK);
            compute(kt & 1);
            if (kt + 1 < KT) sstore((kt + 1) & 1);
            lds_barrier();
        }
        return;
    }

    // Direct-to-LDS loads. Wave w, pass p fills LDS rows (p * NW + w) * RPI
    // + lane / CH, slot lane % CH, with the global chunk that the swizzle
    // puts in that slot. Every call issues A_DMA + B_DMA instructions per
    // wave; past K the loads are out of range and fill zeros.
    const int drow0 = wave * S::RPI + lane / S::CH;
    const int dslot = lane % S::CH;
    // Loads lo .. hi - 1 of the A_DMA + B_DMA of one tile.
    // Loads lo .. hi - 1 of one tile. CHECK: K-chunks at or past K load as
    // zero (the K tail). Without CHECK (K a multiple of BK) a tile at or past
    // K reads whatever follows the rows or zeros past the operand's end; such
    // tiles are prefetches that are never read.
    auto dma_range_t = [&](int stage, int64_t k0, int lo, int hi, auto check) {
        constexpr bool CHECK = decltype(check)::value;
        char* sbase = lds + stage * S::LDS_STAGE;
        const uint32_t kb = (uint32_t)(k0 * S::ESZ);
#pragma unroll
        for (int p = 0; p < S::A_DMA + S::B_DMA; ++p) {
            if (p < lo || p >= hi) continue;
            const bool is_a = p < S::A_DMA;
            const int pp = is_a ? p : p - S::A_DMA;
            const int row = pp * S::NW * S::RPI + drow0;
            const int ch = dslot ^ ((row >> S::SWZ_SHIFT) & (S::CH - 1));
            const uint32_t off = (uint32_t)(row * (is_a ? lda : ldb) * S::ESZ + ch * 16) + kb;
            char* dst = sbase + (is_a ? 0 : S::LDS_A) + (pp * S::NW + wave) * 1024;
            uint32_t o = off;
            if (CHECK) o = (k0 + ch * S::EPC) < K ? off : kOobOffset;
            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                is_a ? rsa : rsb, (__attribute__((address_space(3))) void*)dst, 16, o, 0, 0, 0);
        }
    };
    using Checked = std::integral_constant<bool, true>;
    auto dma_range = [&](int stage, int64_t k0, int lo, int hi) {
        dma_range_t(stage, k0, lo, hi, Checked{});
    };
    auto dma = [&](int stage, int64_t k0) { dma_range(stage, k0, 0, S::A_DMA + S::B_DMA); };
    // At a barrier a wave keeps its last NST - 2 tiles of loads in flight.
    constexpr int VM = (S::NST - 2) * (S::A_DMA + S::B_DMA);

    if (S::SCHED == 6) {
        // Ping-pong. Every wave runs Mem(t), barrier, Comp(t), barrier for
        // t = 0, 1, ...; group 1 passes one extra barrier first and group 0
        // one extra barrier last, so between two barriers one group
        // multiplies while the other loads. Mem(t) issues this wave's share
        // of the loads of tile t + NST - 1 into the stage of tile t - 1,
        // which both groups finished reading before the barrier that
        // precedes it. The barrier right after a wave's Mem(t) sees its share
        // of tile t + 1 landed, before either group's Mem(t + 1) reads it.
        const int group = wave / (S::NW / 2);
        u32x4_t fa[S::KSTEPS][S::MB], fb[S::KSTEPS][S::NB];
        auto mem_phase = [&](int t) {
            const int st = t % S::NST;
            dma(st == 0 ? S::NST - 1 : st - 1, (int64_t)(t + S::NST - 1) * S::BK);
            const char* base = lds + st * S::LDS_STAGE;
#pragma unroll
            for (int kk = 0; kk < S::KSTEPS; ++kk) {
                const uint32_t cofs = (uint32_t)((((kk * 2 + khalf) ^ swz)) * 16);
#pragma unroll
                for (int mb = 0; mb < S::MB; ++mb)
                    fa[kk][mb] = *(const u32x4_t*)(base + a_frag0 + mb * 32 * S::RB + cofs);
#pragma unroll
                for (int nb = 0; nb < S::NB; ++nb)
                    fb[kk][nb] = *(const u32x4_t*)(base + b_frag0 + nb * 32 * S::RB + cofs);
            }
        };
        auto comp_phase = [&]() {
            __builtin_amdgcn_s_setprio(1);
#pragma unroll
            for (int kk = 0; kk < S::KSTEPS; ++kk)
#pragma unroll
                for (int mb = 0; mb < S::MB; ++mb)
#pragma unroll
                    for (int nb = 0; nb < S::NB; ++nb)
                        mfma_kstep<S>(acc.v[mb][nb], fa[kk][mb], fb[kk][nb]);
            __builtin_amdgcn_s_setprio(0);
        };
#pragma unroll
        for (int st = 0; st + 1 < S::NST; ++st) dma(st, (int64_t)st * S::BK);
        wait_barrier<VM>();
        if (group == 1) wait_barrier<VM>();
        for (int t = 0; t < KT; ++t) {
            mem_phase(t);
            wait_barrier<VM>();
            comp_phase();
            wait_barrier<VM>();
        }
        if (group == 0) wait_barrier<VM>();
    } else if constexpr (S::SCHED == 7) {
        // Pair i = tiles 2i (group 0) and 2i + 1 (group 1) in stages 2i % NST
        // and (2i + 1) % NST. Iteration i loads pair i + PA into the stages of
        // pair i - 1; its closing barrier sees pair i + 1 landed.
        constexpr int PA = S::NST / 2 - 1;
        constexpr int VMP = (PA - 1) * 2 * (S::A_DMA + S::B_DMA);
        const int group = wave / S::NWG;
        const int NP = (KT + 1) / 2;
#pragma unroll
        for (int p = 0; p < PA; ++p) {
            dma(2 * p, (int64_t)(2 * p) * S::BK);
            dma(2 * p + 1, (int64_t)(2 * p + 1) * S::BK);
        }
        wait_barrier<VMP>();
        for (int i = 0; i < NP; ++i) {
            const int sp = (2 * (i + PA)) % S::NST;
            dma(sp, (int64_t)(2 * (i + PA)) * S::BK);
            dma(sp + 1, (int64_t)(2 * (i + PA) + 1) * S::BK);
            compute((2 * i + group) % S::NST);
            wait_barrier<VMP>();
        }
        // Every load has landed and every fragment read is done; the stages
        // now carry group 1's accumulators to group 0 (vector j of lane l of
        // wavefront wl at ((wl * NV + j) * 64 + l) * 16 bytes).
        constexpr int NV = S::MB * S::NB * 4;
        static_assert(S::NWG * NV * 64 * 16 <= S::LDS_BYTES, "reduction fits the stages");
        wait_barrier<0>();
        f32x4_t* red = (f32x4_t*)lds + (wl * NV) * 64 + lane;
        if (group == 1) {
#pragma unroll
            for (int j = 0; j < NV; ++j) {
                f32x4_t v;
#pragma unroll
                for (int e = 0; e < 4; ++e) v[e] = acc.v[j / 4 / S::NB][(j / 4) % S::NB][(j % 4) * 4 + e];
                red[j * 64] = v;
            }
        }
        wait_barrier<0>();
        if (group == 0) {
#pragma unroll
            for (int j = 0; j < NV; ++j) {
                const f32x4_t v = red[j * 64];
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    acc.v[j / 4 / S::NB][(j / 4) % S::NB][(j % 4) * 4 + e] =
                        acc.v[j / 4 / S::NB][(j / 4) % S::NB][(j % 4) * 4 + e] + v[e];
            }
        }
        return;
    } else if (S::SCHED == 5) {
        // Tile kt + NST - 1 goes to the stage tile kt - 1 used; the barrier
        // in the middle of tile kt's last k-step sees tile kt + 1 landed
        // and every wave done reading tile kt.
        constexpr int HALF = S::BSPLIT;
#pragma unroll
        for (int st = 0; st + 1 < S::NST; ++st) dma(st, (int64_t)st * S::BK);
        wait_barrier<VM>();
        fload(0, lds, 0);
        int cur = 0;  // stage of tile kt
        for (int kt = 0; kt < KT; ++kt) {
            const char* base = lds + cur * S::LDS_STAGE;
            const int nxt = cur + 1 == S::NST ? 0 : cur + 1;
            dma(cur == 0 ? S::NST - 1 : cur - 1, (int64_t)(kt + S::NST - 1) * S::BK);
#pragma unroll
            for (int kk = 0; kk < S::KSTEPS; ++kk) {
                const int fs = kk & 1;
                if (kk + 1 < S::KSTEPS) {
                    fload(fs ^ 1, base, kk + 1);
                    __builtin_amdgcn_sched_barrier(0);
                    mfma_range(fs, 0, NMF);
                    __builtin_amdgcn_sched_barrier(0);
                } else {
                    mfma_range(fs, 0, HALF);
                    __builtin_amdgcn_sched_barrier(0);
                    wait_barrier<VM>();
                    if (kt + 1 < KT) fload(fs ^ 1, lds + nxt * S::LDS_STAGE, 0);
                    __builtin_amdgcn_sched_barrier(0);
                    mfma_range(fs, HALF, NMF);
                    __builtin_amdgcn_sched_barrier(0);
                }
            }
            cur = nxt;
        }
    } else if constexpr (S::SCHED == 8) {
        // One copy of the loop for a K that is a multiple of BK (no per-load
        // tail check) and one with the check.
        auto sched8 = [&](auto check) {
            // SCHED 5's stage rotation and barrier; the loads of tile
            // kt + NST - 1 (into the stage tile kt - 1 used) are spread over
            // the first DSPREAD k-steps of tile kt, and inside a k-step each
            // MFMA is followed by one fragment read of the next k-step and one
            // load, so the matrix core keeps working while they issue.
            constexpr int HALF = S::BSPLIT;
            constexpr int ND = S::A_DMA + S::B_DMA;
            constexpr int NFR = S::FM + S::FN;
            constexpr int DPK = (ND + S::DSPREAD - 1) / S::DSPREAD;
            static_assert(S::DSPREAD >= 1 && S::DSPREAD < S::KSTEPS, "SCHED 8 load spread");
#pragma unroll
            for (int st = 0; st + 1 < S::NST; ++st)
                dma_range_t(st, (int64_t)st * S::BK, 0, ND, check);
            wait_barrier<VM>();
            fload(0, lds, 0);
            int cur = 0;
            for (int kt = 0; kt < KT; ++kt) {
                const char* base = lds + cur * S::LDS_STAGE;
                const int nxt = cur + 1 == S::NST ? 0 : cur + 1;
                const int dst = cur == 0 ? S::NST - 1 : cur - 1;
                const int64_t k_ld = (int64_t)(kt + S::NST - 1) * S::BK;
#pragma unroll
                for (int kk = 0; kk < S::KSTEPS; ++kk) {
                    const int fs = kk & 1;
                    if (kk + 1 < S::KSTEPS) {
                        const int d_lo = kk * DPK < ND ? kk * DPK : ND;
                        const int d_hi = (kk + 1) * DPK < ND ? (kk + 1) * DPK : ND;
                        // Program order alternates fragment reads and loads
                        // (the loads write LDS, so the scheduler keeps the two
                        // kinds in program order); the MFMAs go between them.
                        constexpr int NJ = NFR > DPK ? NFR : DPK;
#pragma unroll
                        for (int j = 0; j < NJ; ++j) {
                            if (j < NFR) fload_one(fs ^ 1, base, kk + 1, j);
                            if (j < d_hi - d_lo)
                                dma_range_t(dst, k_ld, d_lo + j, d_lo + j + 1, check);
                        }
                        mfma_range(fs, 0, NMF);
#pragma unroll
                        for (int i = 0; i < NMF; ++i) {
                            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                            if (i < NFR) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
                            if (i < d_hi - d_lo) __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);
                        }
                        __builtin_amdgcn_sched_barrier(0);
                    } else {
                        mfma_range(fs, 0, HALF);
                        __builtin_amdgcn_sched_barrier(0);
                        wait_barrier<VM>();
                        // Unconditional (no branch to split the schedule): after
                        // the last tile this reads a stage that is never used.
                        fload(fs ^ 1, lds + nxt * S::LDS_STAGE, 0);
                        mfma_range(fs, HALF, NMF);
#pragma unroll
                        for (int i = HALF; i < NMF; ++i) {
                            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                            if (i - HALF < NFR) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
                        }
                        __builtin_amdgcn_sched_barrier(0);
                    }
                }
                cur = nxt;
            }
        };
        if (K % S::BK == 0)
            sched8(std::integral_constant<bool, false>{});
        else
            sched8(Checked{});
        if constexpr (S::MF16) {
            // 16x16x32 -> 32x32x16 accumulator layout. In a 32x32 block, the
            // 16x16 result D_(sa,sb)[4 (l / 16) + j][l % 16] sits in lane l,
            // element 4 (2 sa + sb) + j; the 32x32x16 layout wants
            // D[8 (i / 4) + 4 (t / 32) + i % 4][t % 32] in lane t, element i.
            // For each pair (elements 8 h + j, 8 h + 4 + j), a permlane16 swap
            // then a permlane32 swap move every value to its lane group, in
            // place.
#pragma unroll
            for (int mb = 0; mb < S::MB; ++mb)
#pragma unroll
                for (int nb = 0; nb < S::NB; ++nb)
#pragma unroll
                    for (int h = 0; h < 2; ++h)
#pragma unroll
                        for (int j = 0; j < 4; ++j) {
                            f32x16_t& c = acc.v[mb][nb];
                            auto r = __builtin_amdgcn_permlane16_swap(
                                __float_as_uint(c[8 * h + j]), __float_as_uint(c[8 * h + 4 + j]),
                                false, false);
                            auto q = __builtin_amdgcn_permlane32_swap(r[0], r[1], false, false);
                            c[8 * h + j] = __uint_as_float(q[0]);
                            c[8 * h + 4 + j] = __uint_as_float(q[1]);
                        }
        }
    } else {
        // Two stages, barrier after each tile.
        dma(0, 0);
        wait_barrier<0>();
        for (int kt = 0; kt < KT; ++kt) {
            if (kt + 1 < KT) dma((kt + 1) & 1, (int64_t)(kt + 1) * S::BK);
            compute(kt & 1);
            wait_barrier<0>();
        }
    }
    // Out-of-range groups may still be writing zeros into LDS.
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt(waitcnt_vm_lgkm0(0));
    asm volatile("" ::: "memory");
}

// Bytes of a row-major operand readable from row `row0` of `rows` (row
// stride ld elements of esz bytes), capped so that every offset the loader
// forms stays below kOobOffset.
__host__ __device__ inline uint32_t operand_bytes(int64_t rows, int64_t row0, int64_t ld,
                                                  int64_t esz = 2) {
    int64_t left = rows - row0;
    if (left <= 0) return 0;
    int64_t b = left * ld * esz;
    return b >= (int64_t)kOobOffset ? kOobOffset - 16u : (uint32_t)b;
}

}  // namespace ncm
