// Multiscale residual vector quantization (encode) on gfx950.
//
// Semantics follow the multiscale residual quantizer of
// research/reference/vq_forward_semantics.md:59-82 (nearest code by
// ||u||^2 + ||c||^2 - 2 u.c, lowest index on ties, codes concatenated level 0
// first, PROJECT.md:279) in its average-pool / nearest-repeat variant, with
// one fixed fp32 operation order that the CPU oracle restates:
//   P_1 = x, P_2s[t] = (P_s[2t] + P_s[2t+1]) * 0.5
//   D_l[t'] = sum over j < l, in order, of C_j[code_j]   (coarse reconstruction)
//   u_l = P_{s_l} - D_l                                  (pooled residual)
//   dist_k = fmaf(-2, dot_fixed(u, c_k), csq_k), code = lowest argmin
// pool(r_l) equals P_{s_l} - D_l in exact arithmetic because the strides are
// non-increasing powers of two, so the full-resolution residual is never
// materialized.
//
// Per level:
//   1. rvq_dist_kernel: bf16 MFMA of the codebook (A, M = codes) against the
//      bf16-rounded residual rows (B, N = rows); the epilogue forms
//      offset + csq_k - 2 S and keeps, per row and per lane chunk of codes,
//      the four smallest as 32-bit keys (distance bits | local code index).
//   2. rvq_rescore_kernel (one wavefront per row): bounds the MFMA pass's
//      error rigorously from the row statistics stored with the bf16 row,
//      rescores every candidate that could be the exact argmin in the fixed
//      fp32 order (bit-identical to the oracle; u in fp32 is formed only for
//      rows with more than one candidate), and writes code, gap, D_{l+1} and
//      the next level's bf16 rows with their statistics (or the
//      reconstruction). A lane chunk whose kept keys cannot be proven to
//      cover every code under the threshold has all of its codes rescored.
#include <algorithm>

#include "gemm_core.h"
#include "rvq.h"

namespace ncm {

// ---------------------------------------------------------------- helpers

template <int NCH>
struct RowVec {
    float v[NCH][4];
};

// Xor-butterfly reductions (offsets 32, 16, 8, 4, 2, 1; same bits in every
// lane), done in VALU.
__device__ __forceinline__ float wave_sum(float v) { return wave_sum_xor(v); }
__device__ __forceinline__ double wave_sum_d(double v) { return wave_sum_xor_d(v); }
__device__ __forceinline__ uint32_t wave_min_u32(uint32_t v) { return wave_min_xor(v); }

// Makes this wavefront's LDS writes visible to its own later LDS reads by
// other lanes: the writes complete (lgkmcnt(0)) and the compiler may not
// move memory operations across this point.
__device__ __forceinline__ void wave_lds_sync() {
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
}

__device__ __forceinline__ uint32_t med3_u32(uint32_t a, uint32_t b, uint32_t c) {
    uint32_t r;
    asm volatile("v_med3_u32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(b), "v"(c));
    return r;
}

// Sorted top-4 of 32-bit keys: insert v, keep the four smallest.
__device__ __forceinline__ void top4_insert(uint32_t (&k)[4], uint32_t v) {
    k[3] = med3_u32(k[2], k[3], v);
    k[2] = med3_u32(k[1], k[2], v);
    k[1] = med3_u32(k[0], k[1], v);
    k[0] = min(k[0], v);
}

__device__ __forceinline__ bool lane_chunk_valid(int64_t d, int m, int lane) {
    return (int64_t)m * 256 + 4 * lane < d;
}

template <int NCH>
__device__ __forceinline__ void load_f32_row(const float* row, int64_t d, int lane,
                                             RowVec<NCH>& r) {
#pragma unroll
    for (int m = 0; m < NCH; ++m) {
        if (lane_chunk_valid(d, m, lane)) {
            const f32x4_t q = *(const f32x4_t*)(row + m * 256 + 4 * lane);
            r.v[m][0] = q[0]; r.v[m][1] = q[1]; r.v[m][2] = q[2]; r.v[m][3] = q[3];
        } else {
            r.v[m][0] = r.v[m][1] = r.v[m][2] = r.v[m][3] = 0.0f;
        }
    }
}

// acc += widen(bf16 row) elementwise (fp32 adds, one per element).
template <int NCH>
__device__ __forceinline__ void add_bf16_row(const uint16_t* row, int64_t d, int lane,
                                             RowVec<NCH>& acc) {
#pragma unroll
    for (int m = 0; m < NCH; ++m) {
        if (lane_chunk_valid(d, m, lane)) {
            const u32x2_t p = *(const u32x2_t*)(row + m * 256 + 4 * lane);
            acc.v[m][0] = acc.v[m][0] + bf16_lo_to_f32(p[0]);
            acc.v[m][1] = acc.v[m][1] + bf16_hi_to_f32(p[0]);
            acc.v[m][2] = acc.v[m][2] + bf16_lo_to_f32(p[1]);
            acc.v[m][3] = acc.v[m][3] + bf16_hi_to_f32(p[1]);
        }
    }
}

// The oracle's ncmo_dot_fixed: lane j accumulates elements 256 m + 4 j + e
// (m ascending, then e) with fmaf from +0, then an xor butterfly (same bits
// in every lane, fp32 addition being commutative).
template <int NCH>
__device__ __forceinline__ float dot_fixed(const RowVec<NCH>& u, const uint16_t* c, int64_t d,
                                           int lane) {
    float acc = 0.0f;
#pragma unroll
    for (int m = 0; m < NCH; ++m) {
        if (lane_chunk_valid(d, m, lane)) {
            const u32x2_t p = *(const u32x2_t*)(c + m * 256 + 4 * lane);
            acc = __builtin_fmaf(u.v[m][0], bf16_lo_to_f32(p[0]), acc);
            acc = __builtin_fmaf(u.v[m][1], bf16_hi_to_f32(p[0]), acc);
            acc = __builtin_fmaf(u.v[m][2], bf16_lo_to_f32(p[1]), acc);
            acc = __builtin_fmaf(u.v[m][3], bf16_hi_to_f32(p[1]), acc);
        }
    }
    return wave_sum(acc);
}

__device__ __forceinline__ int ilog2_pow2(int64_t s) { return 63 - __builtin_clzll((uint64_t)s); }

__device__ __forceinline__ const float* pooled_row_ptr(const RvqGeom& g, const float* x,
                                                       const float* pyr, int level,
                                                       int64_t row) {
    const int64_t s = g.L.stride[level];
    if (s == 1) return x + row * g.d;
    return pyr + g.pyr_off[ilog2_pow2(s)] + row * g.d;
}

// D = sum over j < level (in order, from +0) of C_j[code_j] for one row.
template <int NCH>
__device__ __forceinline__ void coarse_recon(const RvqGeom& g, const uint16_t* cb,
                                             const int32_t* codes, int level, int64_t row,
                                             int lane, RowVec<NCH>& D) {
#pragma unroll
    for (int m = 0; m < NCH; ++m) D.v[m][0] = D.v[m][1] = D.v[m][2] = D.v[m][3] = 0.0f;
    const int64_t s = g.L.stride[level];
    const int64_t per_b = g.t / s;
    const int64_t bb = row / per_b, tp = row % per_b;
    for (int j = 0; j < level; ++j) {
        int32_t k = codes[bb * g.L.total + g.L.offset[j] + (tp * s) / g.L.stride[j]];
        k = k < 0 ? 0 : (k >= g.v ? (int32_t)(g.v - 1) : k);
        add_bf16_row<NCH>(cb + ((int64_t)j * g.v + k) * g.d, g.d, lane, D);
    }
}

struct RowStats {
    float unorm;   // ||u|| (rounded up)
    float dnorm;   // ||u - bf16(u)|| (rounded up)
    double unorm2; // ||u||^2 in f64 (gap reporting)
};

// Writes bf16(u) and returns the norms of u and of its rounding error.
template <int NCH>
__device__ __forceinline__ RowStats write_bf16_row(const RowVec<NCH>& u, int64_t d, int lane,
                                                   uint16_t* dst) {
    float su = 0.0f, sd = 0.0f;
    double su2 = 0.0;
#pragma unroll
    for (int m = 0; m < NCH; ++m) {
        if (lane_chunk_valid(d, m, lane)) {
            uint32_t b[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const float v = u.v[m][e];
                b[e] = bf16_bits_rne(v);
                const float r = v - __uint_as_float(b[e] << 16);
                su = __builtin_fmaf(v, v, su);
                sd = __builtin_fmaf(r, r, sd);
                su2 = __builtin_fma((double)v, (double)v, su2);
            }
            if (dst) {
                u32x2_t o;
                o[0] = b[0] | (b[1] << 16);
                o[1] = b[2] | (b[3] << 16);
                *(u32x2_t*)(dst + m * 256 + 4 * lane) = o;
            }
        }
    }
    RowStats s;
    // 1e-4 relative head-room covers the rounding of the sums.
    s.unorm = sqrtf(wave_sum(su) * 1.0001f);
    s.dnorm = sqrtf(wave_sum(sd) * 1.0001f);
    s.unorm2 = wave_sum_d(su2);
    return s;
}

// Offset that keeps offset + csq_k - 2 S_k >= 0 for every code:
// |S_k| <= ||bf16(u)|| ||c_k|| (1 + d 2^-23) and ||bf16(u)|| <= unorm + dnorm.
__device__ __forceinline__ float row_offset(const RowStats& s, float cmax) {
    return 2.0f * (s.unorm + s.dnorm) * cmax * (1.0f + 1.0f / 1024.0f) + 1e-30f;
}

// ------------------------------------------------------------- pyramid

// Pools `src` rows [R, d] by 2, 4, ..., 2^DEPTH in one pass; dst[k] receives
// the stride-2^(k+1) pool relative to src. A thread owns 4 columns of one
// group of 2^DEPTH consecutive rows (groups never straddle a batch row,
// because t is a multiple of the largest stride).
// The per-encode set-up of one level by one workgroup of NT threads:
// cmax[l] = sqrt(max_k csq[l, k]) (rounded up); zeroes the level's two
// counters (counts[l], counts[levels + l]). Each thread issues its (up to)
// four loads of a pass together, so the workgroup waits for one memory round
// trip per 4 NT codes. The maximum does not depend on the order, so any NT
// gives the same bits.
struct SetupArgs {
    const float* csq;
    int64_t v, levels;
    float* cmax;
    int32_t* counts;
};

template <int NT>
__device__ __forceinline__ void rvq_setup_level(const SetupArgs& sa, int l) {
    const float* row = sa.csq + (int64_t)l * sa.v;
    float m = 0.0f;
    for (int64_t k0 = threadIdx.x; k0 < sa.v; k0 += 4 * NT) {
        float t[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int64_t k = k0 + (int64_t)j * NT;
            t[j] = k < sa.v ? row[k] : 0.0f;
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) m = fmaxf(m, t[j]);
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) m = fmaxf(m, __shfl_xor(m, off, 64));
    __shared__ float red[NT / 64];
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = m;
    __syncthreads();
    if (threadIdx.x == 0) {
        float r = red[0];
        for (int w = 1; w < NT / 64; ++w) r = fmaxf(r, red[w]);
        sa.cmax[l] = sqrtf(r) * 1.00001f;
        sa.counts[l] = 0;
        sa.counts[sa.levels + l] = 0;
    }
}

// Pooling passes of up to seven halvings; the first pass also runs the
// per-encode set-up in its first setup_blocks workgroups (one per level),
// which then finish while the pooling streams.
constexpr int kMaxPyrPass = 7;  // halvings per pyramid pass
template <int DEPTH>
__global__ __launch_bounds__(256) void rvq_pyramid_kernel(const float* __restrict__ src,
                                                          int64_t rows, int64_t d,
                                                          float* __restrict__ dst0,
                                                          float* __restrict__ dst1,
                                                          float* __restrict__ dst2,
                                                          float* __restrict__ dst3,
                                                          float* __restrict__ dst4,
                                                          float* __restrict__ dst5,
                                                          float* __restrict__ dst6,
                                                          SetupArgs sa, int setup_blocks) {
    if ((int)blockIdx.x < setup_blocks) {
        rvq_setup_level<256>(sa, (int)blockIdx.x);
        return;
    }
    constexpr int N = 1 << DEPTH;
    const int64_t q = d / 4;
    const int64_t idx = (int64_t)(blockIdx.x - setup_blocks) * blockDim.x + threadIdx.x;
    const int64_t groups = rows >> DEPTH;
    if (idx >= groups * q) return;
    const int64_t g = idx / q, c = (idx % q) * 4;
    float* dst[kMaxPyrPass] = {dst0, dst1, dst2, dst3, dst4, dst5, dst6};
    // Rows are loaded RB at a time; every loop is unrolled, so the stack
    // level each row reaches is known at compile time.
    constexpr int RB = N < 16 ? N : 16;
    f32x4_t stk[DEPTH];
#pragma unroll
    for (int r0 = 0; r0 < N; r0 += RB) {
        f32x4_t in[RB];
#pragma unroll
        for (int i = 0; i < RB; ++i)
            in[i] = *(const f32x4_t*)(src + ((g << DEPTH) + r0 + i) * d + c);
#pragma unroll
        for (int i = 0; i < RB; ++i) {
            const int r = r0 + i;
            f32x4_t v = in[i];
#pragma unroll
            for (int k = 0; k < DEPTH; ++k) {
                if ((r >> k) & 1) {
                    f32x4_t s;
#pragma unroll
                    for (int e = 0; e < 4; ++e) s[e] = (stk[k][e] + v[e]) * 0.5f;
                    v = s;
                    *(f32x4_t*)(dst[k] + (((g << DEPTH) + r) >> (k + 1)) * d + c) = v;
                } else {
                    stk[k] = v;
                    break;
                }
            }
        }
    }
}

// ------------------------------------------------- per-encode set-up kernel

// The set-up alone (no pyramid pass to carry it: every stride is 1).
constexpr int kSetupThreads = 1024;
__global__ __launch_bounds__(kSetupThreads) void rvq_setup_kernel(SetupArgs sa) {
    rvq_setup_level<kSetupThreads>(sa, (int)blockIdx.x);
}

// ------------------------------------------------------ level-0 prep kernel

struct PrepArgs {
    RvqGeom g;
    const float* x;
    const float* pyr;
    const uint16_t* cb;
    const int32_t* resid_codes;
    const float* cmax;
    uint16_t* ubuf;
    float* rowc;
    RowStats* stats;
    int level;
    int64_t n_rows;
};

// u = P - D for every row of a level; bf16(u) and the row offset.
template <int NCH>
__global__ __launch_bounds__(256) void rvq_prep_kernel(PrepArgs a) {
    const int lane = threadIdx.x & 63;
    const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= a.n_rows) return;
    RowVec<NCH> D, u;
    coarse_recon<NCH>(a.g, a.cb, a.resid_codes, a.level, row, lane, D);
    load_f32_row<NCH>(pooled_row_ptr(a.g, a.x, a.pyr, a.level, row), a.g.d, lane, u);
#pragma unroll
    for (int m = 0; m < NCH; ++m)
#pragma unroll
        for (int e = 0; e < 4; ++e) u.v[m][e] = u.v[m][e] - D.v[m][e];
    const RowStats s = write_bf16_row<NCH>(u, a.g.d, lane, a.ubuf + row * a.g.d);
    if (lane == 0) {
        a.rowc[row] = row_offset(s, a.cmax[a.level]);
        a.stats[row] = s;
    }
}

// ------------------------------------------------------- distance kernel

// Candidate key layout: the distance bits (offset + csq - 2S >= 0, so the
// fp32 pattern orders like the value) with the low `ib` bits replaced by the
// code's index inside its chunk. Chunk = (range, wave row wm): the four
// smallest keys of the codes that one wavefront row holds for a row, over
// both lane halves h; local index = ((tile * MB + mb) * 16 + i) * 2 + h for
// accumulator element i of block mb in tile `tile` of the range.
struct CandGeom {
    int bm;       // codes per tile
    int wm_codes; // codes per wave along M
    int mb;       // 32-code blocks per wave
    int wgm;      // waves along M
    int ntv;      // tiles per range
    int nranges;
    int ib;       // index bits
    int nchunk;   // chunks per row = nranges * wgm
    int mb_log2;  // log2(mb), log2(wgm): both are powers of two
    int wgm_log2;
};

struct DistArgs {
    const uint16_t* cb;   // level codebook [v, d]
    const uint16_t* ubuf; // [n_rows, d]
    const float* csq;     // level [v]
    const float* rowc;    // [n_rows]
    uint32_t* cand;       // [n_rows, nchunk, 4]
    int64_t n_rows, v, d;
    CandGeom cg;
};

// Folds one finished code tile into the running per-row top-4 keys.
// FULL: every code of the tile is < v (no per-value guard).
template <class S, bool FULL>
__device__ __forceinline__ void dist_epilogue(const GemmAcc<S>& acc, const DistArgs& a,
                                              int64_t code0, int tile, int wm, int half,
                                              const float (&rowc)[S::NB], uint32_t imask,
                                              uint32_t (&top)[S::NB][4]) {
#pragma unroll
    for (int mb = 0; mb < S::MB; ++mb) {
        const int64_t cbase = code0 + wm * S::WM + mb * 32 + 4 * half;
        float cs[16];
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const int64_t code = cbase + 8 * (i >> 2) + (i & 3);
            cs[i] = (FULL || code < a.v) ? a.csq[code] : 0.0f;
        }
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const uint32_t local = (uint32_t)(((tile * S::MB + mb) * 16 + i) * 2 + half);
            const bool ok = FULL || (cbase + 8 * (i >> 2) + (i & 3) < a.v);
#pragma unroll
            for (int nb = 0; nb < S::NB; ++nb) {
                const float dist = __builtin_fmaf(acc.v[mb][nb][i], -2.0f, cs[i] + rowc[nb]);
                uint32_t key = (__float_as_uint(dist) & ~imask) | local;
                if (!FULL) key = ok ? key : 0xFFFFFFFFu;
                top4_insert(top[nb], key);
            }
        }
    }
}

constexpr int kDistGroup = 8;

// ONE: each workgroup has one code tile (ntv == 1), so the per-row state
// (offsets, top-4 keys) is created after the main loop and holds no registers
// during it.
template <class S, bool ONE>
__global__ __launch_bounds__(S::NT)
__attribute__((amdgpu_waves_per_eu(S::OCC, S::OCC))) void rvq_dist_kernel(DistArgs a) {
    extern __shared__ __attribute__((aligned(16))) char lds[];
    // XCD-aware grouped order: each XCD receives a contiguous run of logical
    // ids, and a run of kDistGroup x nranges ids covers kDistGroup row tiles
    // (fastest) by every code range, so the 32 workgroups an XCD runs at
    // once share 8 row tiles and 4 code tiles in its L2.
    const int logical = xcd_remap((int)blockIdx.x, (int)gridDim.x);
    const int nr = a.cg.nranges;
    const int row_tiles = (int)gridDim.x / nr;
    const int per_group = kDistGroup * nr;
    const int grp = logical / per_group;
    const int gm = min(kDistGroup, row_tiles - grp * kDistGroup);
    const int in_g = logical - grp * per_group;
    const int rt = grp * kDistGroup + in_g % gm;
    const int range = in_g / gm;
    const int64_t row0 = (int64_t)rt * S::BN;
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int wm = wave % S::WGM;
    const int wn = wave / S::WGM;
    const int half = lane >> 5;
    const uint32_t imask = (1u << a.cg.ib) - 1u;

    auto load_rowc = [&](float (&rowc)[S::NB]) {
#pragma unroll
        for (int nb = 0; nb < S::NB; ++nb) {
            const int64_t r = row0 + wn * S::WN + nb * 32 + (lane & 31);
            rowc[nb] = r < a.n_rows ? a.rowc[r] : 0.0f;
        }
    };
    auto init_top = [&](uint32_t (&top)[S::NB][4]) {
#pragma unroll
        for (int nb = 0; nb < S::NB; ++nb)
#pragma unroll
            for (int j = 0; j < 4; ++j) top[nb][j] = 0xFFFFFFFFu;
    };
    // Lanes l and l + 32 hold the same rows (the two halves of each 8-code
    // group): lanes 0-31 fold the other half's four keys into their own and
    // store one chunk per (range, wave row).
    auto store_top = [&](uint32_t (&top)[S::NB][4]) {
        const int chunk = range * S::WGM + wm;
#pragma unroll
        for (int nb = 0; nb < S::NB; ++nb) {
            uint32_t other[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) other[j] = swap32(top[nb][j])[1];
#pragma unroll
            for (int j = 0; j < 4; ++j) top4_insert(top[nb], other[j]);
        }
#pragma unroll
        for (int nb = 0; nb < S::NB; ++nb) {
            const int64_t r = row0 + wn * S::WN + nb * 32 + (lane & 31);
            if (half == 0 && r < a.n_rows) {
                u32x4_t o;
                o[0] = top[nb][0]; o[1] = top[nb][1]; o[2] = top[nb][2]; o[3] = top[nb][3];
                *(u32x4_t*)(a.cand + (r * a.cg.nchunk + chunk) * 4) = o;
            }
        }
    };

    const uint32_t b_bytes = operand_bytes(a.n_rows, row0, a.d);
    if constexpr (ONE) {
        const int64_t code0 = (int64_t)range * S::BM;
        GemmAcc<S> acc;
        acc.zero();
        gemm_mainloop<S>(a.cb + code0 * a.d, a.d, operand_bytes(a.v, code0, a.d),
                         a.ubuf + row0 * a.d, a.d, b_bytes, a.d, lds, acc);
        float rowc[S::NB];
        load_rowc(rowc);
        uint32_t top[S::NB][4];
        init_top(top);
        if (code0 + S::BM <= a.v)
            dist_epilogue<S, true>(acc, a, code0, 0, wm, half, rowc, imask, top);
        else
            dist_epilogue<S, false>(acc, a, code0, 0, wm, half, rowc, imask, top);
        store_top(top);
    } else {
        float rowc[S::NB];
        load_rowc(rowc);
        uint32_t top[S::NB][4];
        init_top(top);
        for (int tile = 0; tile < a.cg.ntv; ++tile) {
            const int64_t code0 = ((int64_t)range * a.cg.ntv + tile) * S::BM;
            if (code0 >= a.v) break;
            GemmAcc<S> acc;
            acc.zero();
            gemm_mainloop<S>(a.cb + code0 * a.d, a.d, operand_bytes(a.v, code0, a.d),
                             a.ubuf + row0 * a.d, a.d, b_bytes, a.d, lds, acc);
            if (code0 + S::BM <= a.v)
                dist_epilogue<S, true>(acc, a, code0, tile, wm, half, rowc, imask, top);
            else
                dist_epilogue<S, false>(acc, a, code0, tile, wm, half, rowc, imask, top);
        }
        store_top(top);
    }
}

// --------------------------------------------------------- rescore kernel

// Candidate keys per row are read 64 per lane slot: KS slots hold up to
// 16 KS chunks of four keys (KS = 8 for the default tiles, 16 for the small
// levels' 64 x 64 tiles, whose rows have twice as many chunks).
constexpr int kKeySlots = 8;
constexpr int kMaxChunks = kKeySlots * 64 / 4;
constexpr int kKeySlotsWide = 16;
constexpr int kMaxChunksWide = kKeySlotsWide * 64 / 4;

// Per-level arguments of the rescore kernel.
struct RowArgs {
    RvqGeom g;
    const float* x;
    const float* pyr;
    const uint16_t* cb;          // all codebooks [levels, v, d]
    const float* csq;            // all levels [levels, v]
    const int32_t* force_codes;  // nullable: codes that build later residuals
    int32_t* codes;
    float* gap;                  // nullable
    const uint32_t* cand;
    const float* rowc_in;
    const RowStats* stats_in;
    RowStats* stats_out;
    const float* cmax;
    const float* d_in;           // D_l, one row per level l-1 row (level > 0)
    float* d_out;                // D_{l+1}, one row per level-l row (not last level)
    uint16_t* ubuf;              // level l+1 bf16 rows
    float* rowc_out;             // level l+1 offsets
    float* recon;                // last level only, nullable
    int32_t* flag_count;         // this level's counter of rows with an
                                 // incomplete chunk
    int32_t* score_count;        // nullable: this level's counter of rows
                                 // with any exact distance (diagnostics:
                                 // one same-address atomic per such row)
    int level;
    int64_t n_rows;
    int64_t d_div;               // level-l rows per D_l row (s_{l-1} / s_l)
    CandGeom cg;
};

__device__ __forceinline__ int64_t decode_code(const CandGeom& cg, int chunk, uint32_t local) {
    const int half = (int)(local & 1u);
    local >>= 1;
    const int wm = chunk & (cg.wgm - 1);
    const int range = chunk >> cg.wgm_log2;
    const int i = (int)(local & 15u);
    const int mb = (int)((local >> 4) & (uint32_t)(cg.mb - 1));
    const int tile = (int)((local >> 4) >> cg.mb_log2);
    return ((int64_t)range * cg.ntv + tile) * cg.bm + wm * cg.wm_codes + mb * 32 +
           8 * (i >> 2) + 4 * half + (i & 3);
}

struct Best {
    float best, second;
    int32_t code;
};

// Returns true when `code` becomes the best (wave-uniform: every lane holds
// the same distance bits).
__device__ __forceinline__ bool best_update(Best& b, float dist, int32_t code) {
    if (dist < b.best || (dist == b.best && code < b.code)) {
        b.second = b.best;
        b.best = dist;
        b.code = code;
        return true;
    }
    if (dist < b.second) b.second = dist;
    return false;
}

// The bf16 elements of one code row that a lane owns (lane j: elements
// 256 m + 4 j .. + 3), as loaded for a dot product.
template <int NCH>
struct CodeRow {
    u32x2_t p[NCH];
};

template <int NCH>
__device__ __forceinline__ void load_code_row(const uint16_t* c, int64_t d, int lane,
                                              CodeRow<NCH>& r) {
#pragma unroll
    for (int m = 0; m < NCH; ++m)
        if (lane_chunk_valid(d, m, lane)) r.p[m] = *(const u32x2_t*)(c + m * 256 + 4 * lane);
}

// acc += widen(code row) elementwise (fp32 adds, one per element).
template <int NCH>
__device__ __forceinline__ void add_code_row(const CodeRow<NCH>& r, int64_t d, int lane,
                                             RowVec<NCH>& acc) {
#pragma unroll
    for (int m = 0; m < NCH; ++m) {
        if (lane_chunk_valid(d, m, lane)) {
            acc.v[m][0] = acc.v[m][0] + bf16_lo_to_f32(r.p[m][0]);
            acc.v[m][1] = acc.v[m][1] + bf16_hi_to_f32(r.p[m][0]);
            acc.v[m][2] = acc.v[m][2] + bf16_lo_to_f32(r.p[m][1]);
            acc.v[m][3] = acc.v[m][3] + bf16_hi_to_f32(r.p[m][1]);
        }
    }
}

__device__ __forceinline__ float rel_gap(const Best& b, double unorm2) {
    if (!(b.second < INFINITY)) return INFINITY;
    const double e1 = unorm2 + (double)b.best, e2 = unorm2 + (double)b.second;
    return (float)((e2 - e1) / fmax(fabs(e1), 1e-300));
}

// kDotBatch fixed-order dot products at once (all code rows loaded before
// any arithmetic, so one memory round trip serves the batch). Each result
// has the bits of the oracle's ncmo_dot_fixed.
constexpr int kDotBatch = 2;

template <int NCH>
__device__ __forceinline__ void dotn_fixed(const RowVec<NCH>& u,
                                           const uint16_t* const (&c)[kDotBatch], int64_t d,
                                           int lane, float (&out)[kDotBatch],
                                           CodeRow<NCH> (&rows)[kDotBatch]) {
#pragma unroll
    for (int j = 0; j < kDotBatch; ++j) load_code_row<NCH>(c[j], d, lane, rows[j]);
    float acc[kDotBatch];
#pragma unroll
    for (int j = 0; j < kDotBatch; ++j) acc[j] = 0.0f;
#pragma unroll
    for (int m = 0; m < NCH; ++m) {
        if (lane_chunk_valid(d, m, lane)) {
#pragma unroll
            for (int j = 0; j < kDotBatch; ++j) {
                acc[j] = __builtin_fmaf(u.v[m][0], bf16_lo_to_f32(rows[j].p[m][0]), acc[j]);
                acc[j] = __builtin_fmaf(u.v[m][1], bf16_hi_to_f32(rows[j].p[m][0]), acc[j]);
                acc[j] = __builtin_fmaf(u.v[m][2], bf16_lo_to_f32(rows[j].p[m][1]), acc[j]);
                acc[j] = __builtin_fmaf(u.v[m][3], bf16_hi_to_f32(rows[j].p[m][1]), acc[j]);
            }
        }
    }
#pragma unroll
    for (int j = 0; j < kDotBatch; ++j) out[j] = wave_sum(acc[j]);
}

// Exact distances of `n` codes listed in `list` (wave-uniform), folded into
// b; best_row keeps the elements of b's code once it was scored here.
template <int NCH>
__device__ __forceinline__ void score_list(const RowVec<NCH>& u, const uint16_t* cbl,
                                           const float* csql, const int32_t* list, int n,
                                           int64_t d, int lane, Best& b,
                                           CodeRow<NCH>& best_row) {
    for (int i = 0; i < n; i += kDotBatch) {
        int32_t k[kDotBatch];
        const uint16_t* c[kDotBatch];
#pragma unroll
        for (int j = 0; j < kDotBatch; ++j) {
            k[j] = list[i + j < n ? i + j : i];
            c[j] = cbl + (int64_t)k[j] * d;
        }
        float dots[kDotBatch];
        CodeRow<NCH> rows[kDotBatch];
        dotn_fixed<NCH>(u, c, d, lane, dots, rows);
#pragma unroll
        for (int j = 0; j < kDotBatch; ++j)
            if (i + j < n && best_update(b, __builtin_fmaf(-2.0f, dots[j], csql[k[j]]), k[j]))
                best_row = rows[j];
    }
}

// D_l for one row (zero at level 0).
template <int NCH>
__device__ __forceinline__ void load_coarse(const RowArgs& a, int64_t row, int lane,
                                            RowVec<NCH>& D) {
    if (a.level == 0) {
#pragma unroll
        for (int m = 0; m < NCH; ++m) D.v[m][0] = D.v[m][1] = D.v[m][2] = D.v[m][3] = 0.0f;
    } else {
        load_f32_row<NCH>(a.d_in + (row / a.d_div) * a.g.d, a.g.d, lane, D);
    }
}

// Code and gap of a finished row; D_{l+1} and the next level's bf16 rows, or
// the reconstruction at the last level.
// best_row holds the elements of b.code when have_row is true. KEEP_D: D_l
// is still in D (else it is loaded again).
template <int NCH, bool KEEP_D, bool PAIR>
__device__ __forceinline__ void finish_row(const RowArgs& a, int64_t row, const Best& b,
                                          const CodeRow<NCH>& best_row, bool have_row,
                                          double unorm2, int lane, RowVec<NCH>& D,
                                          RowVec<NCH> (&ch)[2]) {
    const RvqGeom& g = a.g;
    const int l = a.level;
    const int64_t d = g.d;
    const int64_t s = g.L.stride[l];
    const int64_t per_b = g.t / s;
    const int64_t bb = row / per_b, tp = row - bb * per_b;
    const int64_t ci = bb * g.L.total + g.L.offset[l] + tp;
    if (lane == 0) {
        a.codes[ci] = b.code;
        if (a.gap) a.gap[ci] = rel_gap(b, unorm2);
    }
    const bool last = l + 1 >= g.L.levels;
    if (last && !a.recon) return;
    int32_t k = a.force_codes ? a.force_codes[ci] : b.code;
    k = k < 0 ? 0 : (k >= g.v ? (int32_t)(g.v - 1) : k);
    if (!KEEP_D) load_coarse<NCH>(a, row, lane, D);
    if (have_row && k == b.code) {
        add_code_row<NCH>(best_row, d, lane, D);  // D_{l+1}
    } else {
        CodeRow<NCH> r;
        load_code_row<NCH>(a.cb + ((int64_t)l * g.v + k) * d, d, lane, r);
        add_code_row<NCH>(r, d, lane, D);
    }
    if (last) {
        // recon[bb, tp * s .. tp * s + s - 1] = D_L
        for (int64_t r = 0; r < s; ++r) {
            float* dst = a.recon + (bb * g.t + tp * s + r) * d;
#pragma unroll
            for (int m = 0; m < NCH; ++m)
                if (lane_chunk_valid(d, m, lane)) {
                    f32x4_t o;
                    o[0] = D.v[m][0]; o[1] = D.v[m][1]; o[2] = D.v[m][2]; o[3] = D.v[m][3];
                    *(f32x4_t*)(dst + m * 256 + 4 * lane) = o;
                }
        }
        return;
    }
    {
        float* dst = a.d_out + row * d;
#pragma unroll
        for (int m = 0; m < NCH; ++m)
            if (lane_chunk_valid(d, m, lane)) {
                f32x4_t o;
                o[0] = D.v[m][0]; o[1] = D.v[m][1]; o[2] = D.v[m][2]; o[3] = D.v[m][3];
                *(f32x4_t*)(dst + m * 256 + 4 * lane) = o;
            }
    }
    const int64_t ratio = PAIR ? 2 : s / g.L.stride[l + 1];
    for (int64_t c = 0; c < ratio; ++c) {
        const int64_t child = row * ratio + c;
        RowVec<NCH> u;
        if constexpr (PAIR)
            u = ch[c];
        else
            load_f32_row<NCH>(pooled_row_ptr(g, a.x, a.pyr, l + 1, child), d, lane, u);
#pragma unroll
        for (int m = 0; m < NCH; ++m)
#pragma unroll
            for (int e = 0; e < 4; ++e) u.v[m][e] = u.v[m][e] - D.v[m][e];
        const RowStats st = write_bf16_row<NCH>(u, d, lane, a.ubuf + child * d);
        if (lane == 0) {
            a.rowc_out[child] = row_offset(st, a.cmax[l + 1]);
            a.stats_out[child] = st;
        }
    }
}

// One wavefront per row. The row's offset and statistics come from the
// kernel that built its bf16 row, so the exact residual u = P_s - D_l is
// formed only when some candidate needs an exact distance.
// KEEP_D: D_l stays in registers from the start to the finish (else it is
// loaded again for each use: d above 2048 at the large levels).
// PAIR: the next level pools by half this level's stride; its two child rows
// are loaded at the start, give P_s = (c0 + c1) * 0.5 (the pyramid's own
// operation, so the pyramid's bits) when u is needed, and the next level's
// rows at the finish.
template <int NCH, int KS, bool KEEP_D, bool PAIR>
__global__ __launch_bounds__(256) void rvq_rescore_kernel(RowArgs a) {
    constexpr int kKeySlots = KS;
    __shared__ int32_t cand_list[4][kKeySlots * 64];
    __shared__ int32_t inc_list[4][kKeySlots * 16];
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int64_t row = (int64_t)blockIdx.x * 4 + wave;
    if (row >= a.n_rows) return;
    const RvqGeom& g = a.g;
    const int l = a.level;
    const int64_t d = g.d;

    RowVec<NCH> u, D;
    RowVec<NCH> ch[2];
    if constexpr (PAIR) {
#pragma unroll
        for (int c = 0; c < 2; ++c)
            load_f32_row<NCH>(pooled_row_ptr(g, a.x, a.pyr, l + 1, 2 * row + c), d, lane, ch[c]);
    }
    if constexpr (KEEP_D) load_coarse<NCH>(a, row, lane, D);
    const int nk = a.cg.nchunk * 4;
    const uint32_t* ck = a.cand + row * (int64_t)nk;
    uint32_t key[kKeySlots];
#pragma unroll
    for (int s = 0; s < kKeySlots; ++s) {
        const int idx = lane + 64 * s;
        key[s] = idx < nk ? ck[idx] : 0xFFFFFFFFu;
    }
    const RowStats st = a.stats_in[row];

    // Rigorous bound E on |key distance - (offset + exact dist)|:
    //   bf16 rounding of u:     2 cmax ||u - bf16(u)||
    //   MFMA fp32 accumulation: 2 cmax d 2^-23 ||bf16(u)||
    //   fixed-order rescore:    2 cmax (d/64 + 7) 2^-23 ||u||
    //   epilogue / final ops:   2^-21 of the largest magnitude involved.
    const float cmax = a.cmax[l];
    const float rowc = a.rowc_in[row];
    const float ub = st.unorm + st.dnorm;
    const float dmag = cmax * cmax + rowc + 2.0f * ub * cmax;
    const float E = 2.0f * cmax *
                        (st.dnorm + (float)d * 0x1p-23f * ub +
                         ((float)(d / 64) + 7.0f) * 0x1p-23f * st.unorm) +
                    dmag * 0x1p-21f + 1e-30f;
    const uint32_t imask = (1u << a.cg.ib) - 1u;
    uint32_t mn = 0xFFFFFFFFu;
#pragma unroll
    for (int s = 0; s < kKeySlots; ++s) mn = min(mn, key[s]);
    mn = wave_min_u32(mn);
    const float m_f = __uint_as_float(mn & ~imask);
    const float eps_q = __uint_as_float((uint32_t)(127 + a.cg.ib - 23) << 23);  // 2^(ib-23)
    // When gaps are reported, codes whose exact relative gap to the best is
    // below ~2e-5 are always rescored, so the reported gap is exact for
    // near-ties. The argmin itself needs only the 2E window: the true
    // nearest code's key is at most 2E above the smallest key.
    const float tau = a.gap ? 2e-5f * (st.unorm * st.unorm + fabsf(m_f - rowc) + 2.0f * E)
                            : 0.0f;
    const float thr = (m_f * (1.0f + eps_q) + 2.0f * E + tau) * (1.0f + 0x1p-20f);

    // Candidates: keys under the threshold. A chunk whose fourth (largest
    // kept) key is under the threshold may hold more codes under it than it
    // kept ("incomplete"): all of its codes are rescored instead of its
    // keys. The four keys of a chunk sit in one lane quad of one slot.
    int32_t* list = cand_list[wave];
    int32_t* inc = inc_list[wave];
    int nsel = 0, ninc = 0;
#pragma unroll
    for (int s = 0; s < kKeySlots; ++s) {
        const int idx = lane + 64 * s;
        const bool valid = idx < nk && key[s] != 0xFFFFFFFFu;
        const bool under = valid && __uint_as_float(key[s] & ~imask) <= thr;
        const bool head = under && (idx & 3) == 3;
        const bool chunk_inc =
            __builtin_amdgcn_update_dpp(0, head ? 1 : 0, 0xFF, 0xF, 0xF, false) != 0;  // quad lane 3
        const bool take = under && !chunk_inc;
        const uint64_t mask = __ballot(take);
        if (take) {
            const int pos = nsel + __builtin_amdgcn_mbcnt_hi((uint32_t)(mask >> 32),
                                                              __builtin_amdgcn_mbcnt_lo((uint32_t)mask, 0));
            list[pos] = (int32_t)decode_code(a.cg, idx >> 2, key[s] & imask);
        }
        nsel += __popcll(mask);
        const uint64_t hmask = __ballot(head);
        if (head) {
            const int pos = ninc + __builtin_amdgcn_mbcnt_hi((uint32_t)(hmask >> 32),
                                                              __builtin_amdgcn_mbcnt_lo((uint32_t)hmask, 0));
            inc[pos] = idx >> 2;
        }
        ninc += __popcll(hmask);
    }
    wave_lds_sync();

    const uint16_t* cbl = a.cb + (int64_t)l * g.v * d;
    const float* csql = a.csq + (int64_t)l * g.v;
    Best b{INFINITY, INFINITY, 0x7FFFFFFF};
    CodeRow<NCH> best_row;
    bool have_row = false;
    if (nsel == 1 && ninc == 0) {
        // One code under the threshold: it is the exact argmin and no other
        // code lies within the near-tie window, so no exact distance is
        // needed (the gap is +inf, as for any single rescored candidate).
        b.code = list[0];
    } else {
        if (a.score_count && lane == 0) atomicAdd(a.score_count, 1);
        // The exact residual, only for rows that need exact distances.
        if constexpr (PAIR) {
#pragma unroll
            for (int m = 0; m < NCH; ++m)
#pragma unroll
                for (int e = 0; e < 4; ++e) u.v[m][e] = (ch[0].v[m][e] + ch[1].v[m][e]) * 0.5f;
        } else {
            load_f32_row<NCH>(pooled_row_ptr(g, a.x, a.pyr, l, row), d, lane, u);
        }
        if constexpr (!KEEP_D) load_coarse<NCH>(a, row, lane, D);
#pragma unroll
        for (int m = 0; m < NCH; ++m)
#pragma unroll
            for (int e = 0; e < 4; ++e) u.v[m][e] = u.v[m][e] - D.v[m][e];
        score_list<NCH>(u, cbl, csql, list, nsel, d, lane, b, best_row);
        have_row = nsel > 0;
    }
    if (ninc > 0) {
        if (lane == 0) atomicAdd(a.flag_count, 1);
        // Every code of each incomplete chunk, listed in LDS then rescored.
        const int nloc = a.cg.ntv * a.cg.mb * 32;
        for (int c = 0; c < ninc; ++c) {
            const int chunk = inc[c];
            for (int base = 0; base < nloc; base += kKeySlots * 64) {
                wave_lds_sync();  // the previous list has been read
                int n = 0;
                for (int off = 0; off < kKeySlots * 64 && base + off < nloc; off += 64) {
                    const int local = base + off + lane;
                    const int64_t code =
                        local < nloc ? decode_code(a.cg, chunk, (uint32_t)local) : g.v;
                    const bool ok = code < g.v;
                    const uint64_t m = __ballot(ok);
                    if (ok) {
                        const int pos = n + __builtin_amdgcn_mbcnt_hi(
                                                (uint32_t)(m >> 32),
                                                __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0));
                        list[pos] = (int32_t)code;
                    }
                    n += __popcll(m);
                }
                wave_lds_sync();
                score_list<NCH>(u, cbl, csql, list, n, d, lane, b, best_row);
                have_row = true;
            }
        }
    }
    finish_row<NCH, KEEP_D, PAIR>(a, row, b, best_row, have_row, st.unorm2, lane, D, ch);
}

// ------------------------------------------------------------ host side

// Distance GEMM tiles (codes x rows), all loading global -> LDS directly
// with two wavefronts per SIMD (SCHED 8 main loop):
//   DistBig    256 x 256, 8 wavefronts, 2 LDS stages: when it gives at least
//              one workgroup per CU;
//   DistMid    256 x 128, 8 wavefronts, 3 stages: when its tiles fill the CUs
//              at least once;
//   DistSmall  128 x 128, 4 wavefronts, 4 stages (deeper prefetch for the
//              latency-bound small grids): at most one workgroup per CU;
//   DistSmall2 128 x 128, 2 stages (64 KB: two workgroups per CU) between.
// DistBig and DistMid share one candidate layout (256 codes per tile, 4
// wavefronts along the codes), DistSmall and DistSmall2 another.
using DistBig = GemmShape<256, 256, 64, 4, 2, 2, 8, true, 2, false, 1, -1, 2>;
// DistBig on 16x16x32 MFMAs (its fragments take 48 more VGPRs: only with one
// code tile per workgroup, when no per-row state lives through the main loop).
using DistBig16 = GemmShape<256, 256, 64, 4, 2, 2, 8, true, 2, false, 1, -1, -1, true>;
using DistMid = GemmShape<256, 128, 64, 4, 2, 2, 8, true, 3, false, 1, -1, -1, true>;
using DistSmall = GemmShape<128, 128, 64, 2, 2, 2, 8, true, 4>;
using DistSmall2 = GemmShape<128, 128, 64, 2, 2, 2, 8, true, 2>;
// DistTiny    64 x 64, 4 wavefronts (32 x 32 each), 4 stages (64 KB: two
//             workgroups per CU): the small levels, whose 128 x 128 grids
//             leave most CUs idle; one code tile per workgroup, 16 candidate
//             key slots per row.
using DistTiny = GemmShape<64, 64, 64, 2, 2, 2, 8, true, 4>;
constexpr int64_t kCus = 256;
// Levels with at most this many rows keep D_l in registers through the
// rescore at any d (their few rows leave occupancy to spare).
constexpr int64_t kSmallLevelRows = 4096;

static int nch_for(int64_t d) {
    const int64_t n = (d + 255) / 256;
    if (n <= 1) return 1;
    if (n <= 2) return 2;
    if (n <= 4) return 4;
    if (n <= 8) return 8;
    return 16;
}

template <int NCH, bool PAIR>
static void launch_rescore_p(const RowArgs* ra, int64_t rows, dim3 grid, hipStream_t st) {
    if (ra->cg.nchunk > kMaxChunks)
        hipLaunchKernelGGL((rvq_rescore_kernel<NCH, kKeySlotsWide, true, PAIR>), grid, dim3(256),
                           0, st, *ra);
    else if (NCH <= 8 || rows <= kSmallLevelRows)
        hipLaunchKernelGGL((rvq_rescore_kernel<NCH, kKeySlots, true, PAIR>), grid, dim3(256), 0,
                           st, *ra);
    else
        hipLaunchKernelGGL((rvq_rescore_kernel<NCH, kKeySlots, false, PAIR>), grid, dim3(256), 0,
                           st, *ra);
}

template <int NCH>
static hipError_t launch_row_kernels(const PrepArgs* pa, const RowArgs* ra, int64_t rows,
                                     hipStream_t st) {
    const dim3 grid((unsigned)((rows + 3) / 4));
    if (pa) {
        hipLaunchKernelGGL(rvq_prep_kernel<NCH>, grid, dim3(256), 0, st, *pa);
        return hipGetLastError();
    }
    const int l = ra->level;
    const bool pair = NCH <= 8 && l + 1 < ra->g.L.levels &&
                      ra->g.L.stride[l] == 2 * ra->g.L.stride[l + 1];
    if (pair)
        launch_rescore_p<NCH, NCH <= 8>(ra, rows, grid, st);
    else
        launch_rescore_p<NCH, false>(ra, rows, grid, st);
    return hipGetLastError();
}

// Level-0 prep (pa) or a level's rescore (ra).
static hipError_t launch_rows(int nch, const PrepArgs* pa, const RowArgs* ra, int64_t rows,
                              hipStream_t st) {
    switch (nch) {
        case 1: return launch_row_kernels<1>(pa, ra, rows, st);
        case 2: return launch_row_kernels<2>(pa, ra, rows, st);
        case 4: return launch_row_kernels<4>(pa, ra, rows, st);
        case 8: return launch_row_kernels<8>(pa, ra, rows, st);
        default: return launch_row_kernels<16>(pa, ra, rows, st);
    }
}

template <class S>
static CandGeom cand_geom_t(int64_t n_rows, int64_t v, int max_chunks = kMaxChunks) {
    CandGeom cg{};
    cg.bm = S::BM;
    cg.wm_codes = S::WM;
    cg.mb = S::MB;
    cg.wgm = S::WGM;
    const int64_t tiles_v = (v + S::BM - 1) / S::BM;
    const int64_t rt = (n_rows + S::BN - 1) / S::BN;
    const int64_t max_ranges = max_chunks / (S::WGM * 2);
    int64_t nr = std::min<int64_t>(max_ranges, tiles_v);
    // Large levels: fewer, longer ranges (less candidate traffic).
    while (nr > 8 && rt * nr > 2048) nr /= 2;
    cg.ntv = (int)((tiles_v + nr - 1) / nr);
    cg.nranges = (int)((tiles_v + cg.ntv - 1) / cg.ntv);
    const int locals = cg.ntv * S::MB * 32;
    int ib = 0;
    while ((1 << ib) < locals) ++ib;
    cg.ib = ib;
    cg.nchunk = cg.nranges * S::WGM;
    static_assert((S::MB & (S::MB - 1)) == 0 && (S::WGM & (S::WGM - 1)) == 0,
                  "candidate decoding shifts by log2(MB) and log2(WGM)");
    cg.mb_log2 = __builtin_ctz(S::MB);
    cg.wgm_log2 = __builtin_ctz(S::WGM);
    return cg;
}

enum DistKind { kDistBig, kDistMid, kDistSmall, kDistSmall2, kDistTiny };

static int64_t dist_grid(const CandGeom& cg, int64_t n_rows, int64_t bn) {
    return (n_rows + bn - 1) / bn * cg.nranges;
}

static DistKind dist_kind(int64_t n_rows, int64_t v) {
    if (dist_grid(cand_geom_t<DistBig>(n_rows, v), n_rows, DistBig::BN) >= kCus) return kDistBig;
    if (dist_grid(cand_geom_t<DistMid>(n_rows, v), n_rows, DistMid::BN) >= kCus) return kDistMid;
    const int64_t small = dist_grid(cand_geom_t<DistSmall>(n_rows, v), n_rows, DistSmall::BN);
    if (small <= kCus / 2 &&
        cand_geom_t<DistTiny>(n_rows, v, kMaxChunksWide).ntv == 1)
        return kDistTiny;
    if (small <= kCus) return kDistSmall;
    return kDistSmall2;
}

static CandGeom cand_geom(int64_t n_rows, int64_t v) {
    switch (dist_kind(n_rows, v)) {
        case kDistBig: return cand_geom_t<DistBig>(n_rows, v);
        case kDistMid: return cand_geom_t<DistMid>(n_rows, v);
        case kDistTiny: return cand_geom_t<DistTiny>(n_rows, v, kMaxChunksWide);
        default: return cand_geom_t<DistSmall>(n_rows, v);
    }
}

template <class S, bool ONE>
static hipError_t launch_dist_t(const DistArgs& da, hipStream_t st) {
    auto kern = rvq_dist_kernel<S, ONE>;
    static bool attr_set = false;
    if (!attr_set) {
        hipError_t e = hipFuncSetAttribute((const void*)kern,
                                           hipFuncAttributeMaxDynamicSharedMemorySize,
                                           S::LDS_BYTES);
        if (e != hipSuccess) return e;
        attr_set = true;
    }
    const int64_t rt = (da.n_rows + S::BN - 1) / S::BN;
    hipLaunchKernelGGL(kern, dim3((unsigned)(rt * da.cg.nranges)), dim3(S::NT), S::LDS_BYTES,
                       st, da);
    return hipGetLastError();
}

template <class S>
static hipError_t launch_dist(const DistArgs& da, hipStream_t st) {
    return da.cg.ntv == 1 ? launch_dist_t<S, true>(da, st) : launch_dist_t<S, false>(da, st);
}

static size_t align256(size_t v) { return (v + 255) & ~size_t(255); }

// Workspace layout of one encode (byte offsets from a 256-byte aligned base).
struct RvqLayout {
    size_t pyr, u, d0, d1, rc0, rc1, st0, st1, cand, cmax, fc, total;
};

// Fills the geometry and the workspace layout; NCM_E_SHAPE if the rows are
// wider than the row kernels hold or the strides need more pyramid levels
// than the geometry holds.
static int rvq_layout(int64_t b, int64_t t, int64_t d, int64_t levels, const int32_t* strides,
                      int64_t v, RvqGeom& g, RvqLayout& lay) {
    if (d > kMaxEncodeWidth) return NCM_E_SHAPE;
    g = RvqGeom{};
    g.b = b; g.t = t; g.d = d; g.v = v;
    g.L = make_level_table(t, levels, strides);
    const int64_t smax = strides[0];
    int jmax = 0;
    while ((int64_t(1) << jmax) < smax) ++jmax;
    if (jmax >= kMaxPyr) return NCM_E_SHAPE;
    size_t off = 0;
    auto carve = [&](size_t bytes) { size_t o = off; off = align256(off + bytes); return o; };
    int64_t pyr_floats = 0;
    for (int j = 1; j <= jmax; ++j) {
        g.pyr_off[j] = pyr_floats;
        pyr_floats += b * (t >> j) * d;
    }
    int64_t max_rows = 0, max_cand = 0;
    for (int64_t l = 0; l < levels; ++l) {
        const int64_t n = b * (t / strides[l]);
        max_rows = std::max(max_rows, n);
        max_cand = std::max(max_cand, n * (int64_t)cand_geom(n, v).nchunk * 4);
    }
    lay.pyr = carve((size_t)pyr_floats * 4);
    lay.u = carve((size_t)max_rows * d * 2);
    // Level l (l + 1 < levels) writes D_{l+1} to dbuf[(l + 1) & 1]: dbuf[1]
    // from level 0 on (two or more levels), dbuf[0] from level 1 on.
    lay.d0 = carve(levels > 2 ? (size_t)max_rows * d * 4 : 0);
    lay.d1 = carve(levels > 1 ? (size_t)max_rows * d * 4 : 0);
    lay.rc0 = carve((size_t)max_rows * 4);
    lay.rc1 = carve((size_t)max_rows * 4);
    lay.st0 = carve((size_t)max_rows * sizeof(RowStats));
    lay.st1 = carve((size_t)max_rows * sizeof(RowStats));
    lay.cand = carve((size_t)max_cand * 4);
    lay.cmax = carve((size_t)levels * 4);
    // Per level: rows with an incomplete chunk, then rows with any exact
    // distance.
    lay.fc = carve((size_t)levels * 2 * 4);
    lay.total = off;
    return NCM_OK;
}

int rvq_workspace_bytes(int64_t b, int64_t t, int64_t d, int64_t levels, const int32_t* strides,
                        int64_t v, size_t* bytes) {
    RvqGeom g;
    RvqLayout lay;
    const int rc = rvq_layout(b, t, d, levels, strides, v, g, lay);
    if (rc) return rc;
    *bytes = lay.total;
    return NCM_OK;
}

int rvq_encode(ncm_ctx_t* ctx, const float* x, int64_t b, int64_t t, int64_t d, int64_t levels,
               const int32_t* strides, const uint16_t* codebooks, const float* csq, int64_t v,
               int32_t* codes, float* recon, float* gap, const int32_t* force_codes,
               int64_t* n_flagged, RvqCounts* counts) {
    size_t bytes = 0;
    int rc = rvq_workspace_bytes(b, t, d, levels, strides, v, &bytes);
    if (rc) return rc;
    void* ws = nullptr;
    rc = ncm_ctx_workspace(ctx, bytes, &ws);
    if (rc) return rc;
    return rvq_encode_ws(ncm_ctx_stream(ctx), ws, bytes, x, b, t, d, levels, strides, codebooks,
                         csq, v, codes, recon, gap, force_codes, n_flagged, counts);
}

int rvq_encode_ws(hipStream_t st, void* ws, size_t ws_bytes, const float* x, int64_t b,
                  int64_t t, int64_t d, int64_t levels, const int32_t* strides,
                  const uint16_t* codebooks, const float* csq, int64_t v, int32_t* codes,
                  float* recon, float* gap, const int32_t* force_codes, int64_t* n_flagged,
                  RvqCounts* counts) {
    RvqGeom g;
    RvqLayout lay;
    int rc = rvq_layout(b, t, d, levels, strides, v, g, lay);
    if (rc) return rc;
    if (ws_bytes < lay.total || ((uintptr_t)ws & 255)) return NCM_E_ARG;
    const int64_t smax = strides[0];
    int jmax = 0;
    while ((int64_t(1) << jmax) < smax) ++jmax;
    char* W = (char*)ws;
    float* pyr = (float*)(W + lay.pyr);
    uint16_t* ubuf = (uint16_t*)(W + lay.u);
    float* rowc[2] = {(float*)(W + lay.rc0), (float*)(W + lay.rc1)};
    RowStats* stats[2] = {(RowStats*)(W + lay.st0), (RowStats*)(W + lay.st1)};
    uint32_t* cand = (uint32_t*)(W + lay.cand);
    float* cmax = (float*)(W + lay.cmax);
    int32_t* fcount = (int32_t*)(W + lay.fc);  // [levels] flagged, [levels] scored
    // D_{l+1} (coarse reconstruction) is written by level l into dbuf[(l+1)&1].
    float* dbuf[2] = {(float*)(W + lay.d0), (float*)(W + lay.d1)};

    const SetupArgs sa{csq, v, levels, cmax, fcount};
    hipError_t e = hipSuccess;
    if (jmax == 0) {
        hipLaunchKernelGGL(rvq_setup_kernel, dim3((unsigned)levels), dim3(kSetupThreads), 0, st,
                           sa);
        e = hipGetLastError();
        if (e != hipSuccess) return NCM_E_HIP;
    }

    // Pyramid, in passes of up to seven halvings; the first pass carries the
    // set-up in its first `levels` workgroups.
    {
        int j0 = 0;
        while (j0 < jmax) {
            const int depth = std::min(kMaxPyrPass, jmax - j0);
            const float* src = j0 == 0 ? x : pyr + g.pyr_off[j0];
            const int64_t rows = b * (t >> j0);
            float* dst[kMaxPyrPass] = {};
            for (int k = 0; k < depth; ++k) dst[k] = pyr + g.pyr_off[j0 + k + 1];
            const int64_t work = (rows >> depth) * (d / 4);
            const int sb = j0 == 0 ? (int)levels : 0;
            const dim3 grid((unsigned)((work + 255) / 256 + sb));
#define NCM_PYR(D)                                                                            \
    hipLaunchKernelGGL(rvq_pyramid_kernel<D>, grid, dim3(256), 0, st, src, rows, d, dst[0],    \
                       dst[1], dst[2], dst[3], dst[4], dst[5], dst[6], sa, sb)
            switch (depth) {
                case 1: NCM_PYR(1); break;
                case 2: NCM_PYR(2); break;
                case 3: NCM_PYR(3); break;
                case 4: NCM_PYR(4); break;
                case 5: NCM_PYR(5); break;
                case 6: NCM_PYR(6); break;
                default: NCM_PYR(7); break;
            }
#undef NCM_PYR
            e = hipGetLastError();
            if (e != hipSuccess) return NCM_E_HIP;
            j0 += depth;
        }
    }

    const int nch = nch_for(d);

    // Level 0 rows.
    {
        PrepArgs pa{};
        pa.g = g; pa.x = x; pa.pyr = pyr; pa.cb = codebooks; pa.resid_codes = codes;
        pa.cmax = cmax; pa.ubuf = ubuf; pa.rowc = rowc[0]; pa.stats = stats[0]; pa.level = 0;
        pa.n_rows = b * (t / strides[0]);
        e = launch_rows(nch, &pa, nullptr, pa.n_rows, st);
        if (e != hipSuccess) return NCM_E_HIP;
    }

    for (int64_t l = 0; l < levels; ++l) {
        const int64_t n = b * (t / strides[l]);
        const CandGeom cg = cand_geom(n, v);
        DistArgs da{};
        da.cb = codebooks + l * v * d;
        da.ubuf = ubuf;
        da.csq = csq + l * v;
        da.rowc = rowc[l & 1];
        da.cand = cand;
        da.n_rows = n; da.v = v; da.d = d;
        da.cg = cg;
        switch (dist_kind(n, v)) {
            case kDistBig:
                e = da.cg.ntv == 1 ? launch_dist_t<DistBig16, true>(da, st)
                                   : launch_dist_t<DistBig, false>(da, st);
                break;
            case kDistMid: e = launch_dist<DistMid>(da, st); break;
            case kDistSmall: e = launch_dist<DistSmall>(da, st); break;
            case kDistTiny: e = launch_dist_t<DistTiny, true>(da, st); break;
            default: e = launch_dist<DistSmall2>(da, st); break;
        }
        if (e != hipSuccess) return NCM_E_HIP;

        RowArgs ra{};
        ra.g = g; ra.x = x; ra.pyr = pyr; ra.cb = codebooks; ra.csq = csq;
        ra.force_codes = force_codes; ra.codes = codes; ra.gap = gap;
        ra.cand = cand; ra.rowc_in = rowc[l & 1]; ra.cmax = cmax;
        ra.stats_in = stats[l & 1]; ra.stats_out = stats[(l + 1) & 1];
        ra.d_in = l > 0 ? dbuf[l & 1] : nullptr;
        ra.d_out = l + 1 < levels ? dbuf[(l + 1) & 1] : nullptr;
        ra.d_div = l > 0 ? strides[l - 1] / strides[l] : 1;
        ra.ubuf = ubuf; ra.rowc_out = rowc[(l + 1) & 1];
        ra.recon = l + 1 == levels ? recon : nullptr;
        ra.flag_count = fcount + l;
        ra.score_count = counts ? fcount + levels + l : nullptr;
        ra.level = (int)l; ra.n_rows = n; ra.cg = cg;
        e = launch_rows(nch, nullptr, &ra, n, st);
        if (e != hipSuccess) return NCM_E_HIP;
    }

    if (n_flagged || counts) {
        int32_t host[2 * kMaxLevels];
        e = hipMemcpyAsync(host, fcount, levels * 2 * 4, hipMemcpyDeviceToHost, st);
        if (e == hipSuccess) e = hipStreamSynchronize(st);
        if (e != hipSuccess) return NCM_E_HIP;
        int64_t s = 0;
        for (int64_t l = 0; l < levels; ++l) s += host[l];
        if (n_flagged) *n_flagged = s;
        if (counts) {
            counts->levels = levels;
            for (int64_t l = 0; l < levels; ++l) {
                counts->flagged[l] = host[l];
                counts->scored[l] = host[levels + l];
            }
        }
    }
    return NCM_OK;
}

}  // namespace ncm
