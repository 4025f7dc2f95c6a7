// The upstream VQ-VAE tokenizer's inference forward on gfx950, float32
// throughout (the quantizer casts to float32, vq_forward_semantics.md:49;
// research/reference/vq_forward_semantics.md describes the PyTorch module,
// research/converter/wmt14_tokenizer_keys.md the released WMT14 instance).
//
// Activations are [B, L, D] (position-major, channel-contiguous). Every
// convolution is a GEMM on the fp32 MFMA (gemm_mainloop with the 128x128x32
// fp32 tile):
//   * kernel = stride = s convs of the level-0 cascade: [B L / s, s D] is a
//     reshape of [B L, D], so the A operand is the activation itself;
//   * their transposed convs: [B n, D] x [s D, D]^T = [B n, s D], a reshape
//     of [B n s, D];
//   * Phi's kernel-3, padding-1 conv: the upsampled codes live in a padded
//     buffer hpad [B, L + 2, D] whose first and last row of each sequence
//     are zero, so rows t - 1, t, t + 1 are one contiguous 3 D span and the
//     A operand is an overlapping view (row m at hpad + m D, lda = D, K =
//     3 D); virtual rows that straddle two sequences are computed and
//     dropped (2 of every L + 2).
// The nearest-code search is one GEMM per level, [B n, D] x [V, D]^T, whose
// epilogue turns each product into csq - 2 u.e and keeps the per-row
// minimum as a (distance, index) 64-bit key with atomicMin: the lowest
// index wins ties, as torch.argmin does.
#include <algorithm>
#include <cstdlib>
#include <cstring>

#include "gemm_core.h"
#include "linear.h"
#include "status.h"
#include "vq_tok.h"

namespace ncm {

namespace {

// 128 x 128 x 16 fp32 tile, 4 wavefronts of 64 x 64, two LDS stages (32 KB):
// four workgroups per CU, 118 VGPRs (measured faster than 32-deep K tiles with
// two workgroups per CU, deeper pipelines and 8-wavefront tiles).
using VtTile = GemmShape<128, 128, 16, 2, 2, 4, 5, true, 2, true>;
constexpr int kNT = 256;

enum { kEpiStage = 0, kEpiPhi = 1, kEpiDist = 2 };

struct VtEpi {
    // kEpiStage: y = act(acc + bias[n % bias_len]) (+ res, [M, N], may be
    // y); bias NULL: none; act 1: exact GELU. pad_len > 0 stores flat row
    // R = (m N + n) / D of [rows, D] at padded row R + 2 (R / pad_len) + 1.
    const float* bias;
    int64_t bias_len;
    float* y;
    int64_t pad_len;
    int64_t d;
    const float* res;
    int act;
    // kEpiPhi: Q = (1 - ratio) h + ratio (acc + bias); zhat (+)= Q; r -= Q.
    const float* hpad;
    float* zhat;
    float* r;
    float ratio;
    int64_t seq;   // L
    int first;     // zhat = Q instead of zhat += Q
    // kEpiDist: keys[row] = min(keys[row], key(csq[n] - 2 acc, n)).
    const float* csq;
    unsigned long long* keys;
};

// Order-preserving map of a float onto uint32 (NaN -> 0, the smallest: a NaN
// distance wins, as in torch.argmin), paired with the code index.
__device__ __forceinline__ unsigned long long dist_key(float v, int64_t col) {
    uint32_t b = __float_as_uint(v);
    b = (b & 0x80000000u) ? ~b : (b | 0x80000000u);
    if (v != v) b = 0;
    return ((unsigned long long)b << 32) | (uint32_t)col;
}

// Exact GELU (nn.GELU's default): x Phi(x) with the device library's erff.
__device__ __forceinline__ float gelu_exact(float x) {
    return 0.5f * x * (1.0f + erff(x * 0.70710678118654752f));
}

__device__ __forceinline__ float stage_value(const VtEpi& ep, float acc, int64_t n) {
    const float v = ep.bias ? acc + ep.bias[n % ep.bias_len] : acc;
    return ep.act == 1 ? gelu_exact(v) : v;
}

__device__ __forceinline__ unsigned long long shfl_xor_u64(unsigned long long v, int m) {
    const uint32_t lo = __shfl_xor((uint32_t)v, m);
    const uint32_t hi = __shfl_xor((uint32_t)(v >> 32), m);
    return ((unsigned long long)hi << 32) | lo;
}

template <class S, int EPI>
__global__ __launch_bounds__(S::NT)
__attribute__((amdgpu_waves_per_eu(S::OCC, S::OCC))) void vt_gemm_kernel(
    const float* __restrict__ a, int64_t lda, int64_t a_rows, const float* __restrict__ w,
    int64_t M, int64_t K, int64_t N, int tiles_n, int group_m, VtEpi ep) {
    extern __shared__ __attribute__((aligned(16))) char lds[];
    const int logical = xcd_remap((int)blockIdx.x, (int)gridDim.x);
    const int per_group = group_m * tiles_n;
    const int g = logical / per_group;
    const int tiles_m = (int)((M + S::BM - 1) / S::BM);
    const int gm = min(group_m, tiles_m - g * group_m);
    const int in_g = logical % per_group;
    const int tm = g * group_m + in_g % gm;
    const int tn = in_g / gm;
    const int64_t m0 = (int64_t)tm * S::BM;
    const int64_t n0 = (int64_t)tn * S::BN;

    GemmAcc<S> acc;
    acc.zero();
    gemm_mainloop<S>((const char*)a + m0 * lda * 4, lda, operand_bytes(a_rows, m0, lda, 4),
                     (const char*)w + n0 * K * 4, K, operand_bytes(N, n0, K, 4), K, lds, acc);

    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int wm = wave % S::WGM;
    const int wn = wave / S::WGM;

    if constexpr (EPI == kEpiDist) {
        // Per row: the minimum key over this wavefront's columns. A lane
        // holds 16 rows per 32-row block (element i: row 8 (i / 4) + 4 (lane /
        // 32) + i % 4) of one column per 32-column block; the 32 lanes of a
        // half share the rows. Transposed reduction over those 32 lanes: at
        // each xor step a lane keeps half of its rows and sends the other
        // half to its partner, so 16 rows take 8 + 4 + 2 + 1 exchanges; the
        // last step (xor 1) pairs lanes that hold the same row. Lane q ends
        // with row i = q / 2 (even lanes issue the atomic).
        const int q = lane & 31;
#pragma unroll
        for (int mb = 0; mb < S::MB; ++mb) {
            unsigned long long k16[16];
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                unsigned long long best = ~0ull;
#pragma unroll
                for (int nb = 0; nb < S::NB; ++nb) {
                    const int64_t n = n0 + wn * S::WN + nb * 32 + q;
                    if (n < N) {
                        const unsigned long long k =
                            dist_key(ep.csq[n] - 2.0f * acc.v[mb][nb][i], n);
                        best = k < best ? k : best;
                    }
                }
                k16[i] = best;
            }
#pragma unroll
            for (int half = 8; half >= 1; half >>= 1) {
                // xor 2 * half: bit b of q chooses which half of the rows stays.
                const bool up = (q & (2 * half)) != 0;
#pragma unroll
                for (int t = 0; t < half; ++t) {
                    const unsigned long long send = up ? k16[t] : k16[t + half];
                    const unsigned long long keep = up ? k16[t + half] : k16[t];
                    const unsigned long long recv = shfl_xor_u64(send, 2 * half);
                    k16[t] = recv < keep ? recv : keep;
                }
            }
            const unsigned long long o = shfl_xor_u64(k16[0], 1);
            const unsigned long long best = o < k16[0] ? o : k16[0];
            const int i = q >> 1;
            const int64_t m = m0 + wm * S::WM + mb * 32 + 8 * (i >> 2) + 4 * (lane >> 5) + (i & 3);
            if ((q & 1) == 0 && m < M && best != ~0ull) atomicMin(ep.keys + m, best);
        }
        return;
    }

    auto store4 = [&](int64_t m, int64_t n, const float (&v)[4]) {
        if constexpr (EPI == kEpiStage) {
            int64_t dst = m * N + n;
            if (ep.pad_len > 0) {
                const int64_t row = dst / ep.d;
                dst = (row + 2 * (row / ep.pad_len) + 1) * ep.d + dst % ep.d;
            }
            f32x4_t o;
#pragma unroll
            for (int j = 0; j < 4; ++j) o[j] = stage_value(ep, v[j], n + j);
            if (ep.res) o += *(const f32x4_t*)(ep.res + dst);
            *(f32x4_t*)(ep.y + dst) = o;
        } else {
            // Virtual row m = b (L + 2) + t; t >= L straddles two sequences.
            const int64_t b = m / (ep.seq + 2);
            const int64_t t = m - b * (ep.seq + 2);
            if (t >= ep.seq) return;
            const f32x4_t h = *(const f32x4_t*)(ep.hpad + (m + 1) * N + n);
            const int64_t o = (b * ep.seq + t) * N + n;
            f32x4_t q;
#pragma unroll
            for (int j = 0; j < 4; ++j)
                q[j] = (1.0f - ep.ratio) * h[j] + ep.ratio * (v[j] + ep.bias[n + j]);
            if (ep.first) {
                *(f32x4_t*)(ep.zhat + o) = q;
            } else {
                f32x4_t z = *(const f32x4_t*)(ep.zhat + o);
                *(f32x4_t*)(ep.zhat + o) = z + q;
            }
            if (ep.r) {
                f32x4_t rv = *(const f32x4_t*)(ep.r + o);
                *(f32x4_t*)(ep.r + o) = rv - q;
            }
        }
    };

    if (n0 + S::BN <= N) {
        // Whole tile in range along N: each lane stores 4 consecutive columns
        // of one row after a quad transpose of the D fragment.
        const int q = lane & 3;
        const int col4 = (lane & 31) & ~3;
        const int hrow = 4 * (lane >> 5) + q;
#pragma unroll
        for (int nb = 0; nb < S::NB; ++nb) {
            const int64_t ncol = n0 + wn * S::WN + nb * 32 + col4;
#pragma unroll
            for (int mb = 0; mb < S::MB; ++mb) {
#pragma unroll
                for (int blk = 0; blk < 4; ++blk) {
                    float v[4];
#pragma unroll
                    for (int j = 0; j < 4; ++j) v[j] = acc.v[mb][nb][4 * blk + j];
                    quad_transpose4(v, q);
                    const int64_t m = m0 + wm * S::WM + mb * 32 + 8 * blk + hrow;
                    if (m < M) store4(m, ncol, v);
                }
            }
        }
        return;
    }
    // N tail: one element per lane and row (N % 4 == 0, so a 4-column group
    // never straddles N; the 4 lanes of a group store one element each).
#pragma unroll
    for (int nb = 0; nb < S::NB; ++nb) {
        const int64_t n = n0 + wn * S::WN + nb * 32 + (lane & 31);
        if (n >= N) continue;
#pragma unroll
        for (int mb = 0; mb < S::MB; ++mb) {
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const int64_t m =
                    m0 + wm * S::WM + mb * 32 + 8 * (i >> 2) + 4 * (lane >> 5) + (i & 3);
                if (m >= M) continue;
                const float v = acc.v[mb][nb][i];
                if constexpr (EPI == kEpiStage) {
                    int64_t dst = m * N + n;
                    if (ep.pad_len > 0) {
                        const int64_t row = dst / ep.d;
                        dst = (row + 2 * (row / ep.pad_len) + 1) * ep.d + dst % ep.d;
                    }
                    const float o = stage_value(ep, v, n);
                    ep.y[dst] = ep.res ? ep.res[dst] + o : o;
                } else {
                    const int64_t b = m / (ep.seq + 2);
                    const int64_t t = m - b * (ep.seq + 2);
                    if (t >= ep.seq) continue;
                    const float h = ep.hpad[(m + 1) * N + n];
                    const int64_t o = (b * ep.seq + t) * N + n;
                    const float qv = (1.0f - ep.ratio) * h + ep.ratio * (v + ep.bias[n]);
                    ep.zhat[o] = ep.first ? qv : ep.zhat[o] + qv;
                    if (ep.r) ep.r[o] = ep.r[o] - qv;
                }
            }
        }
    }
}

template <int EPI>
hipError_t launch_vt_gemm(const float* a, int64_t lda, int64_t a_rows, const float* w, int64_t M,
                          int64_t K, int64_t N, const VtEpi& ep, hipStream_t st) {
    using S = VtTile;
    auto kern = vt_gemm_kernel<S, EPI>;
    static bool attr_set = false;
    if (!attr_set) {
        hipError_t e = hipFuncSetAttribute((const void*)kern,
                                           hipFuncAttributeMaxDynamicSharedMemorySize,
                                           S::LDS_BYTES);
        if (e != hipSuccess) return e;
        attr_set = true;
    }
    if (M <= 0 || N <= 0) return hipSuccess;
    const int tiles_m = (int)((M + S::BM - 1) / S::BM);
    const int tiles_n = (int)((N + S::BN - 1) / S::BN);
    const int group_m = tiles_m < 4 ? tiles_m : 4;
    hipLaunchKernelGGL(kern, dim3(tiles_m * tiles_n), dim3(S::NT), S::LDS_BYTES, st, a, lda,
                       a_rows, w, M, K, N, tiles_n, group_m, ep);
    return hipGetLastError();
}

__device__ __forceinline__ float block_sum256(float v, float* red) {
    v = wave_sum_xor(v);
    const int wave = threadIdx.x >> 6;
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[wave] = v;
    __syncthreads();
    return red[0] + red[1] + red[2] + red[3];
}

// GroupNorm(G, D, affine=False) of one (sequence, group) per workgroup over
// [B, L, D]: biased statistics over L positions x D / G channels, two passes
// (mean, then the squared deviations). EMBED: the input row t of sequence b
// is wte[ids[b L + t]] + wpe[t] (the encoder in eval mode,
// vq_forward_semantics.md:38-44). y may equal x; y2 (optional) gets a copy.
template <bool EMBED>
__global__ __launch_bounds__(kNT) void vt_group_norm_kernel(const float* x, const int32_t* ids,
                                                            const float* wte, const float* wpe,
                                                            float* y, float* y2, int64_t L,
                                                            int64_t D, int G, float eps) {
    __shared__ float red[4];
    const int g = blockIdx.x;
    const int64_t b = blockIdx.y;
    const int64_t cg = D / G;
    const int64_t c4n = cg / 4;
    const int64_t n4 = L * c4n;
    auto src = [&](int64_t i, int64_t& off) -> f32x4_t {
        const int64_t t = i / c4n;
        const int64_t c = g * cg + 4 * (i - t * c4n);
        off = (b * L + t) * D + c;
        if constexpr (EMBED) {
            const f32x4_t e = *(const f32x4_t*)(wte + (int64_t)ids[b * L + t] * D + c);
            const f32x4_t p = *(const f32x4_t*)(wpe + t * D + c);
            return e + p;
        } else {
            return *(const f32x4_t*)(x + off);
        }
    };
    float s = 0.0f;
    for (int64_t i = threadIdx.x; i < n4; i += kNT) {
        int64_t off;
        const f32x4_t v = src(i, off);
        s += (v[0] + v[1]) + (v[2] + v[3]);
    }
    const float cnt = (float)(L * cg);
    const float mean = block_sum256(s, red) / cnt;
    float q = 0.0f;
    for (int64_t i = threadIdx.x; i < n4; i += kNT) {
        int64_t off;
        const f32x4_t v = src(i, off);
#pragma unroll
        for (int j = 0; j < 4; ++j) q += (v[j] - mean) * (v[j] - mean);
    }
    const float var = block_sum256(q, red) / cnt;
    const float inv = 1.0f / sqrtf(var + eps);
    for (int64_t i = threadIdx.x; i < n4; i += kNT) {
        int64_t off;
        const f32x4_t v = src(i, off);
        f32x4_t o;
#pragma unroll
        for (int j = 0; j < 4; ++j) o[j] = (v[j] - mean) * inv;
        *(f32x4_t*)(y + off) = o;
        if (y2) *(f32x4_t*)(y2 + off) = o;
    }
}

// F.interpolate(mode="area") from L to n positions: u[b, j] = mean of r over
// [floor(j L / n), ceil((j + 1) L / n)), summed in position order.
__global__ __launch_bounds__(kNT) void vt_area_pool_kernel(const float* __restrict__ r,
                                                           float* __restrict__ u, int64_t B,
                                                           int64_t L, int64_t n, int64_t D) {
    const int64_t d4 = D / 4;
    const int64_t total = B * n * d4;
    for (int64_t i = blockIdx.x * (int64_t)kNT + threadIdx.x; i < total;
         i += (int64_t)gridDim.x * kNT) {
        const int64_t c = (i % d4) * 4;
        const int64_t bj = i / d4;
        const int64_t j = bj % n;
        const int64_t b = bj / n;
        const int64_t s0 = (j * L) / n;
        const int64_t s1 = ((j + 1) * L + n - 1) / n;
        f32x4_t acc = {0.0f, 0.0f, 0.0f, 0.0f};
        for (int64_t t = s0; t < s1; ++t) acc += *(const f32x4_t*)(r + (b * L + t) * D + c);
        const float k = (float)(s1 - s0);
        f32x4_t o;
#pragma unroll
        for (int j2 = 0; j2 < 4; ++j2) o[j2] = acc[j2] / k;
        *(f32x4_t*)(u + bj * D + c) = o;
    }
}

// The code of (sequence b, position j) of a level: from the search keys (low
// 32 bits) or from caller codes, clamped to [0, V) either way. stride and
// offset also address the codes output of vt_codes_up_kernel.
struct CodeSrc {
    const unsigned long long* keys;  // [B, n] or NULL
    const int32_t* codes;            // caller codes [B, stride] (+ offset) or NULL
    int64_t stride, offset, v;
    __device__ __forceinline__ int64_t get(int64_t b, int64_t j, int64_t n) const {
        int64_t k = keys ? (int64_t)(uint32_t)keys[b * n + j] : codes[b * stride + offset + j];
        return k < 0 ? 0 : (k >= v ? v - 1 : k);
    }
};

// MODE 0: linear upsample (F.interpolate mode="linear", align_corners
// False) of the level's code vectors from n to L positions into the padded
// buffer's interior rows; MODE 1: n == L, the code vectors themselves into
// the interior rows; MODE 2: the code vectors densely, [B n, D] (the input of
// the level-0 up cascade). codes_out (optional): the codes, [B, stride] at
// offset.
template <int MODE>
__global__ __launch_bounds__(kNT) void vt_codes_up_kernel(CodeSrc src, const float* __restrict__ e,
                                                          float* __restrict__ out,
                                                          int32_t* codes_out, int64_t B, int64_t n,
                                                          int64_t L, int64_t D) {
    const int64_t d4 = D / 4;
    const int64_t rows = MODE == 2 ? n : L;
    const int64_t total = B * rows * d4;
    const float scale = (float)n / (float)L;
    const int64_t gid0 = blockIdx.x * (int64_t)kNT + threadIdx.x;
    if (codes_out) {
        for (int64_t i = gid0; i < B * n; i += (int64_t)gridDim.x * kNT)
            codes_out[(i / n) * src.stride + src.offset + i % n] = (int32_t)src.get(i / n, i % n, n);
    }
    for (int64_t i = gid0; i < total; i += (int64_t)gridDim.x * kNT) {
        const int64_t c = (i % d4) * 4;
        const int64_t bt = i / d4;
        const int64_t t = bt % rows;
        const int64_t b = bt / rows;
        f32x4_t h;
        if (MODE == 0) {
            float s = scale * ((float)t + 0.5f) - 0.5f;
            s = s < 0.0f ? 0.0f : s;
            const int64_t i0 = (int64_t)s;
            const int64_t i1 = i0 + (i0 < n - 1 ? 1 : 0);
            const float l1 = s - (float)i0;
            const float l0 = 1.0f - l1;
            const f32x4_t a = *(const f32x4_t*)(e + src.get(b, i0, n) * D + c);
            const f32x4_t a2 = *(const f32x4_t*)(e + src.get(b, i1, n) * D + c);
#pragma unroll
            for (int j = 0; j < 4; ++j) h[j] = l0 * a[j] + l1 * a2[j];
        } else {
            h = *(const f32x4_t*)(e + src.get(b, t, n) * D + c);
        }
        const int64_t orow = MODE == 2 ? bt : b * (L + 2) + t + 1;
        *(f32x4_t*)(out + orow * D + c) = h;
    }
}

// Q = h (no Phi): zhat (+)= h, r -= h, from the padded buffer's interior.
__global__ __launch_bounds__(kNT) void vt_add_up_kernel(const float* __restrict__ hpad,
                                                        float* zhat, float* r, int64_t B,
                                                        int64_t L, int64_t D, int first) {
    const int64_t d4 = D / 4;
    const int64_t total = B * L * d4;
    for (int64_t i = blockIdx.x * (int64_t)kNT + threadIdx.x; i < total;
         i += (int64_t)gridDim.x * kNT) {
        const int64_t c = (i % d4) * 4;
        const int64_t bt = i / d4;
        const int64_t b = bt / L;
        const f32x4_t h = *(const f32x4_t*)(hpad + (bt + 2 * b + 1) * D + c);
        f32x4_t* zp = (f32x4_t*)(zhat + bt * D + c);
        *zp = first ? h : *zp + h;
        if (r) {
            f32x4_t* rp = (f32x4_t*)(r + bt * D + c);
            *rp = *rp - h;
        }
    }
}

// Zero the first and last row of every sequence of the padded buffer.
__global__ __launch_bounds__(kNT) void vt_pad_rows_kernel(float* hpad, int64_t B, int64_t L,
                                                          int64_t D) {
    const int64_t total = B * 2 * D;
    for (int64_t i = blockIdx.x * (int64_t)kNT + threadIdx.x; i < total;
         i += (int64_t)gridDim.x * kNT) {
        const int64_t c = i % D;
        const int64_t k = (i / D) % 2;
        const int64_t b = i / (2 * D);
        hpad[(b * (L + 2) + k * (L + 1)) * D + c] = 0.0f;
    }
}

// Squared norm of every codebook row, summed in dimension order by one
// thread per row (the rows of all levels in one launch).
struct CbTable {
    const float* cb[NCM_VQ_TOK_MAX_LEVELS];
    int64_t off[NCM_VQ_TOK_MAX_LEVELS + 1];
};

__global__ __launch_bounds__(kNT) void vt_csq_kernel(CbTable tab, int levels, float* csq,
                                                     int64_t D) {
    const int64_t total = tab.off[levels];
    for (int64_t i = blockIdx.x * (int64_t)kNT + threadIdx.x; i < total;
         i += (int64_t)gridDim.x * kNT) {
        int l = 0;
        while (i >= tab.off[l + 1]) ++l;
        const float* row = tab.cb[l] + (i - tab.off[l]) * D;
        float s = 0.0f;
        for (int64_t c = 0; c < D; c += 4) {
            const f32x4_t x = *(const f32x4_t*)(row + c);
            s += x[0] * x[0];
            s += x[1] * x[1];
            s += x[2] * x[2];
            s += x[3] * x[3];
        }
        csq[i] = s;
    }
}

__global__ __launch_bounds__(kNT) void vt_fill_u64_kernel(unsigned long long* p, int64_t n,
                                                          unsigned long long v) {
    for (int64_t i = blockIdx.x * (int64_t)kNT + threadIdx.x; i < n; i += (int64_t)gridDim.x * kNT)
        p[i] = v;
}

// Conv weight repack: Conv1d (out = c, in = c, k): dst[o, j c + i] =
// src[o, i, j]; ConvTranspose1d (in = c, out = c, k): dst[j c + o, i] =
// src[i, o, j].
__global__ __launch_bounds__(kNT) void vt_pack_conv_kernel(const float* __restrict__ src,
                                                           float* __restrict__ dst, int64_t c,
                                                           int64_t k, int transposed) {
    const int64_t total = c * c * k;
    for (int64_t e = blockIdx.x * (int64_t)kNT + threadIdx.x; e < total;
         e += (int64_t)gridDim.x * kNT) {
        if (!transposed) {
            const int64_t o = e / (k * c);
            const int64_t rem = e % (k * c);
            const int64_t j = rem / c;
            const int64_t i = rem % c;
            dst[e] = src[(o * c + i) * k + j];
        } else {
            const int64_t row = e / c;  // j c + o
            const int64_t i = e % c;
            const int64_t j = row / c;
            const int64_t o = row % c;
            dst[e] = src[(i * c + o) * k + j];
        }
    }
}

unsigned grid_for(int64_t work) {
    int64_t g = (work + kNT - 1) / kNT;
    if (g < 1) g = 1;
    if (g > 65536) g = 65536;
    return (unsigned)g;
}

#define VT_TRY(x)                            \
    do {                                     \
        hipError_t e_ = (x);                 \
        if (e_ != hipSuccess) return e_;     \
    } while (0)

struct Ws {
    int64_t B, L, D, nsum, max_n, casc_rows, vsum;
    float* r;
    float* hpad;
    float* u;
    float* c0;
    float* c1;
    float* zhat;
    float* csq;
    unsigned long long* keys;
    int32_t* ids;
};

size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

// Level 0 through the conv cascade (an empty cascade is the identity, as an
// empty nn.Sequential is: then level 0 is handled like any other level).
bool learned(const ncm_vq_tok_t& t) { return t.learned_level0 && t.n_stages > 0; }

// Workspace carve-up (also its size when base is NULL).
size_t carve(const ncm_vq_tok_t& t, int64_t B, bool need_zhat, char* base, Ws* w) {
    const int64_t L = t.level_len[t.n_levels - 1], D = t.embed_dim;
    int64_t nsum = 0, max_n = 0, vsum = 0;
    for (int l = 0; l < t.n_levels; ++l) {
        nsum += t.level_len[l];
        vsum += t.level_vocab[l];
        if (t.level_len[l] < L && t.level_len[l] > max_n) max_n = t.level_len[l];
    }
    // Cascade ping-pong buffers: the largest intermediate is the first down
    // stage's output (L / s0 rows per sequence) or the up stage before the
    // last (L / s_last rows).
    int64_t casc = t.level_len[0];
    if (learned(t)) {
        casc = std::max(L / t.stage_stride[0], L / t.stage_stride[t.n_stages - 1]);
        casc = std::max(casc, t.level_len[0]);
    }
    size_t off = 0;
    auto take = [&](size_t bytes) {
        const size_t o = off;
        off += align256(bytes);
        return base ? base + o : nullptr;
    };
    char* r = take((size_t)(B * L * D) * 4);
    char* hp = take((size_t)(B * (L + 2) * D) * 4);
    char* u = take((size_t)(B * std::max<int64_t>(max_n, 1) * D) * 4);
    char* c0 = take((size_t)(B * casc * D) * 4);
    char* c1 = take((size_t)(B * casc * D) * 4);
    char* zh = need_zhat ? take((size_t)(B * L * D) * 4) : nullptr;
    char* csq = take((size_t)vsum * 4);
    char* keys = take((size_t)(B * nsum) * 8);
    char* ids = take((size_t)(B * L) * 4);
    if (w) {
        w->B = B; w->L = L; w->D = D; w->nsum = nsum; w->max_n = max_n; w->casc_rows = casc;
        w->vsum = vsum;
        w->r = (float*)r; w->hpad = (float*)hp; w->u = (float*)u; w->c0 = (float*)c0;
        w->c1 = (float*)c1; w->zhat = (float*)zh; w->csq = (float*)csq;
        w->keys = (unsigned long long*)keys; w->ids = (int32_t*)ids;
    }
    return off;
}

hipError_t group_norm(const float* x, float* y, float* y2, int64_t B, int64_t L, int64_t D, int G,
                      float eps, hipStream_t st) {
    hipLaunchKernelGGL(vt_group_norm_kernel<false>, dim3(G, (unsigned)B), dim3(kNT), 0, st, x,
                       nullptr, nullptr, nullptr, y, y2, L, D, G, eps);
    return hipGetLastError();
}

hipError_t stage_gemm(const float* x, const float* w, const float* bias, float* y, int64_t M,
                      int64_t K, int64_t N, int64_t bias_len, int64_t pad_len, int64_t D,
                      hipStream_t st) {
    VtEpi ep{};
    ep.bias = bias; ep.bias_len = bias_len; ep.y = y; ep.pad_len = pad_len; ep.d = D;
    return launch_vt_gemm<kEpiStage>(x, K, M, w, M, K, N, ep, st);
}

// Level 0's down cascade: r [B, L, D] -> out [B, L / prod(s), D].
hipError_t cascade_down(const ncm_vq_tok_t& t, const Ws& w, const float* r, float* out,
                        hipStream_t st) {
    const int64_t D = w.D;
    const float* x = r;
    int64_t len = w.L;
    for (int i = 0; i < t.n_stages; ++i) {
        const int64_t s = t.stage_stride[i];
        const bool last = i == t.n_stages - 1;
        float* y = last ? out : ((i & 1) ? w.c1 : w.c0);
        len /= s;
        VT_TRY(stage_gemm(x, t.down_weight[i], t.down_bias[i], y, w.B * len, s * D, D, D, 0, D,
                          st));
        if ((t.cascade_norm && !last) || (t.cascade_norm_final && last))
            VT_TRY(group_norm(y, y, nullptr, w.B, len, D, t.groups, t.group_eps, st));
        x = y;
    }
    return hipSuccess;
}

// Level 0's up cascade: q [B, n0, D] -> the padded buffer's interior rows.
hipError_t cascade_up(const ncm_vq_tok_t& t, const Ws& w, const float* q, hipStream_t st) {
    const int64_t D = w.D;
    const float* x = q;
    int64_t len = t.level_len[0];
    for (int i = 0; i < t.n_stages; ++i) {
        const int64_t s = t.stage_stride[i];
        const bool last = i == t.n_stages - 1;
        float* y = last ? w.hpad : ((i & 1) ? w.c1 : w.c0);
        VT_TRY(stage_gemm(x, t.up_weight[i], t.up_bias[i], y, w.B * len, D, s * D, D,
                          last ? w.L : 0, D, st));
        len *= s;
        if (t.cascade_norm && !last)
            VT_TRY(group_norm(y, y, nullptr, w.B, len, D, t.groups, t.group_eps, st));
        x = y;
    }
    return hipSuccess;
}

// Q_l = Phi_l(hpad interior) added into zhat (first level: stored) and
// subtracted from r (NULL: not kept).
hipError_t apply_resi(const ncm_vq_tok_t& t, const Ws& w, int level, float* zhat, float* r,
                      hipStream_t st) {
    const int64_t B = w.B, L = w.L, D = w.D;
    if (!t.resi_weight[level]) {
        hipLaunchKernelGGL(vt_add_up_kernel, dim3(grid_for(B * L * D / 4)), dim3(kNT), 0, st,
                           w.hpad, zhat, r, B, L, D, level == 0 ? 1 : 0);
        return hipGetLastError();
    }
    VtEpi ep{};
    ep.bias = t.resi_bias[level]; ep.hpad = w.hpad; ep.zhat = zhat; ep.r = r;
    ep.ratio = t.resi_ratio; ep.seq = L; ep.first = level == 0 ? 1 : 0;
    const int64_t rows = B * (L + 2);
    return launch_vt_gemm<kEpiPhi>(w.hpad, D, rows, t.resi_weight[level], rows - 2, 3 * D, D, ep,
                                   st);
}

// Rebuild the level's upsampled code vectors (into hpad) from `src`;
// codes_out (optional) receives the codes.
hipError_t level_up(const ncm_vq_tok_t& t, const Ws& w, int level, const CodeSrc& src,
                    int32_t* codes_out, hipStream_t st) {
    const int64_t B = w.B, L = w.L, D = w.D, n = t.level_len[level];
    const float* e = t.codebook[level];
    if (level == 0 && learned(t)) {
        hipLaunchKernelGGL(vt_codes_up_kernel<2>, dim3(grid_for(B * n * D / 4)), dim3(kNT), 0, st,
                           src, e, w.u, codes_out, B, n, L, D);
        VT_TRY(hipGetLastError());
        return cascade_up(t, w, w.u, st);
    }
    if (n == L)
        hipLaunchKernelGGL(vt_codes_up_kernel<1>, dim3(grid_for(B * L * D / 4)), dim3(kNT), 0, st,
                           src, e, w.hpad, codes_out, B, n, L, D);
    else
        hipLaunchKernelGGL(vt_codes_up_kernel<0>, dim3(grid_for(B * L * D / 4)), dim3(kNT), 0, st,
                           src, e, w.hpad, codes_out, B, n, L, D);
    return hipGetLastError();
}

hipError_t quantize_body(const ncm_vq_tok_t& t, const Ws& w, int32_t* codes, float* zhat,
                         hipStream_t st) {
    const int64_t B = w.B, L = w.L, D = w.D;
    CbTable tab;
    tab.off[0] = 0;
    for (int l = 0; l < t.n_levels; ++l) {
        tab.cb[l] = t.codebook[l];
        tab.off[l + 1] = tab.off[l] + t.level_vocab[l];
    }
    hipLaunchKernelGGL(vt_csq_kernel, dim3(grid_for(w.vsum)), dim3(kNT), 0, st, tab, t.n_levels,
                       w.csq, D);
    VT_TRY(hipGetLastError());
    hipLaunchKernelGGL(vt_fill_u64_kernel, dim3(grid_for(B * w.nsum)), dim3(kNT), 0, st, w.keys,
                       B * w.nsum, ~0ull);
    VT_TRY(hipGetLastError());
    hipLaunchKernelGGL(vt_pad_rows_kernel, dim3(grid_for(B * 2 * D)), dim3(kNT), 0, st, w.hpad, B,
                       L, D);
    VT_TRY(hipGetLastError());

    int64_t off = 0, voff = 0;
    for (int l = 0; l < t.n_levels; ++l) {
        const int64_t n = t.level_len[l], V = t.level_vocab[l];
        const float* u;
        if (l == 0 && learned(t)) {
            VT_TRY(cascade_down(t, w, w.r, w.u, st));
            u = w.u;
        } else if (n == L) {
            u = w.r;
        } else {
            hipLaunchKernelGGL(vt_area_pool_kernel, dim3(grid_for(B * n * D / 4)), dim3(kNT), 0,
                               st, w.r, w.u, B, L, n, D);
            VT_TRY(hipGetLastError());
            u = w.u;
        }
        VtEpi ep{};
        ep.csq = w.csq + voff;
        ep.keys = w.keys + B * off;
        VT_TRY(launch_vt_gemm<kEpiDist>(u, D, B * n, t.codebook[l], B * n, D, V, ep, st));
        CodeSrc src{w.keys + B * off, nullptr, w.nsum, off, V};
        VT_TRY(level_up(t, w, l, src, codes ? codes : nullptr, st));
        // codes_out addressing: [B, nsum] at offset `off`.
        VT_TRY(apply_resi(t, w, l, zhat, w.r, st));
        off += n;
        voff += V;
    }
    return hipSuccess;
}

// ------------------------------------------------------------------ decoder
// The VQ-VAE decoder in eval mode (models/vae.py:198-258,
// vq_forward_semantics.md:84-94): one pre-LN block (bidirectional attention
// with per-head RMSNorm on q and k, a GELU MLP), ln_f, the output layer.

// LayerNorm of one row per wavefront: (x - mean) / sqrt(var + eps) * w (+ b),
// biased variance, two passes over the row (models/vae.py:6-13).
__global__ __launch_bounds__(kNT) void vt_layer_norm_kernel(const float* __restrict__ x,
                                                            const float* __restrict__ w,
                                                            const float* __restrict__ bias,
                                                            float* __restrict__ y, int64_t rows,
                                                            int64_t D, float eps) {
    const int64_t row = blockIdx.x * (int64_t)(kNT / 64) + (threadIdx.x >> 6);
    if (row >= rows) return;
    const int lane = threadIdx.x & 63;
    const float* xr = x + row * D;
    float s = 0.0f;
    for (int64_t c = 4 * lane; c < D; c += 256) {
        const f32x4_t v = *(const f32x4_t*)(xr + c);
        s += (v[0] + v[1]) + (v[2] + v[3]);
    }
    const float mean = wave_sum_xor(s) / (float)D;
    float q = 0.0f;
    for (int64_t c = 4 * lane; c < D; c += 256) {
        const f32x4_t v = *(const f32x4_t*)(xr + c);
#pragma unroll
        for (int j = 0; j < 4; ++j) q += (v[j] - mean) * (v[j] - mean);
    }
    const float inv = 1.0f / sqrtf(wave_sum_xor(q) / (float)D + eps);
    for (int64_t c = 4 * lane; c < D; c += 256) {
        const f32x4_t v = *(const f32x4_t*)(xr + c);
        const f32x4_t wv = *(const f32x4_t*)(w + c);
        f32x4_t o;
#pragma unroll
        for (int j = 0; j < 4; ++j) o[j] = (v[j] - mean) * inv * wv[j];
        if (bias) o += *(const f32x4_t*)(bias + c);
        *(f32x4_t*)(y + row * D + c) = o;
    }
}

// Per-head RMSNorm of q and k in place (models/vae.py:16-26, :60-62):
// x / sqrt(mean(x^2) + eps) * w over each head_dim slice; one wavefront per
// (row, head) of q (blockIdx.y 0) or k (1). qkv rows are [q | k | v], 3 D.
__global__ __launch_bounds__(64) void vt_qk_norm_kernel(float* qkv, const float* __restrict__ wq,
                                                        const float* __restrict__ wk, int64_t D,
                                                        int heads, int hd, float eps) {
    const int64_t row = blockIdx.x;
    const int which = blockIdx.y / heads;
    const int h = blockIdx.y % heads;
    const int lane = threadIdx.x;
    float* p = qkv + row * 3 * D + which * D + (int64_t)h * hd;
    const float* w = which ? wk : wq;
    float s = 0.0f;
    for (int d = lane; d < hd; d += 64) s += p[d] * p[d];
    const float inv = 1.0f / sqrtf(wave_sum_xor(s) / (float)hd + eps);
    for (int d = lane; d < hd; d += 64) p[d] = p[d] * inv * w[d];
}

// Bidirectional softmax attention, one wavefront per (query, head,
// sequence): scores q.k / sqrt(hd) for every key (lane = key), the maximum,
// exp and their sum, then out[d] = sum_j p_j v_j[d] / sum (lane = d).
// Scores in LDS (up to kAttnMaxT keys).
constexpr int kAttnMaxT = 4096;
__global__ __launch_bounds__(64) void vt_attention_kernel(const float* __restrict__ qkv,
                                                          float* __restrict__ out, int64_t T,
                                                          int64_t D, int hd, float scale) {
    __shared__ float sc[kAttnMaxT];
    __shared__ float qs[256];
    const int64_t t = blockIdx.x;
    const int h = blockIdx.y;
    const int64_t b = blockIdx.z;
    const int lane = threadIdx.x;
    const float* base = qkv + b * T * 3 * D;
    const float* q = base + t * 3 * D + (int64_t)h * hd;
    for (int d = lane; d < hd; d += 64) qs[d] = q[d];
    __syncthreads();
    float mx = -__builtin_inff();
    for (int64_t j = lane; j < T; j += 64) {
        const float* k = base + j * 3 * D + D + (int64_t)h * hd;
        float dot = 0.0f;
        for (int d = 0; d < hd; d += 4) {
            const f32x4_t kv = *(const f32x4_t*)(k + d);
            dot += qs[d] * kv[0];
            dot += qs[d + 1] * kv[1];
            dot += qs[d + 2] * kv[2];
            dot += qs[d + 3] * kv[3];
        }
        const float v = dot * scale;
        sc[j] = v;
        mx = fmaxf(mx, v);
    }
    // wavefront maximum
    for (int off = 32; off >= 1; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off));
    float sum = 0.0f;
    for (int64_t j = lane; j < T; j += 64) {
        const float e = expf(sc[j] - mx);
        sc[j] = e;
        sum += e;
    }
    sum = wave_sum_xor(sum);
    __syncthreads();
    const float inv = 1.0f / sum;
    for (int d = lane; d < hd; d += 64) {
        float acc = 0.0f;
        for (int64_t j = 0; j < T; ++j)
            acc += sc[j] * base[j * 3 * D + 2 * D + (int64_t)h * hd + d];
        out[(b * T + t) * D + (int64_t)h * hd + d] = acc * inv;
    }
}

}  // namespace

size_t vq_tok_workspace_bytes(const ncm_vq_tok_t& t, int64_t batch, bool need_zhat) {
    return carve(t, batch, need_zhat, nullptr, nullptr);
}

hipError_t vq_tok_pack_conv(const float* src, float* dst, int64_t c, int64_t k, int transposed,
                            hipStream_t st) {
    hipLaunchKernelGGL(vt_pack_conv_kernel, dim3(grid_for(c * c * k)), dim3(kNT), 0, st, src, dst,
                       c, k, transposed);
    return hipGetLastError();
}

hipError_t vq_tok_encode(const ncm_vq_tok_t& t, const int32_t* ids_host, const float* latent_in,
                         int64_t batch, int32_t* codes, float* zhat, float* latent_out, void* ws,
                         hipStream_t st) {
    Ws w;
    carve(t, batch, zhat == nullptr, (char*)ws, &w);
    float* zh = zhat ? zhat : w.zhat;
    const int64_t L = w.L, D = w.D;
    if (ids_host) {
        VT_TRY(hipMemcpyAsync(w.ids, ids_host, sizeof(int32_t) * batch * L, hipMemcpyHostToDevice,
                              st));
        hipLaunchKernelGGL(vt_group_norm_kernel<true>, dim3(t.groups, (unsigned)batch), dim3(kNT),
                           0, st, nullptr, w.ids, t.wte, t.wpe, w.r, latent_out, L, D, t.groups,
                           t.group_eps);
        VT_TRY(hipGetLastError());
    } else {
        VT_TRY(hipMemcpyAsync(w.r, latent_in, sizeof(float) * batch * L * D,
                              hipMemcpyDeviceToDevice, st));
    }
    return quantize_body(t, w, codes, zh, st);
}

size_t vq_tok_decoder_workspace_bytes(const ncm_vq_tok_t& t, int64_t batch) {
    const int64_t M = batch * t.level_len[t.n_levels - 1], D = t.embed_dim;
    // x, h (D each), qkv (3 D), attention output (D), MLP hidden (4 D)
    return align256((size_t)(M * D) * 4) * 3 + align256((size_t)(M * 3 * D) * 4) +
           align256((size_t)(M * 4 * D) * 4);
}

hipError_t vq_tok_decode(const ncm_vq_tok_t& t, const ncm_vq_tok_decoder_t& dec, const float* zhat,
                         int64_t batch, float* logits, void* ws, hipStream_t st) {
    const int64_t L = t.level_len[t.n_levels - 1], D = t.embed_dim, M = batch * L;
    const int64_t C = t.in_vocab;
    char* p = (char*)ws;
    auto take = [&](int64_t floats) {
        float* q = (float*)p;
        p += align256((size_t)floats * 4);
        return q;
    };
    float* x = take(M * D);
    float* h = take(M * D);
    float* a = take(M * D);
    float* qkv = take(M * 3 * D);
    float* f = take(M * 4 * D);
    auto gemm = [&](const float* in, const float* w, const float* bias, float* y, int64_t K,
                    int64_t N, const float* res, int act) {
        VtEpi ep{};
        ep.bias = bias; ep.bias_len = N; ep.y = y; ep.d = N; ep.res = res; ep.act = act;
        return launch_vt_gemm<kEpiStage>(in, K, M, w, M, K, N, ep, st);
    };
    auto ln = [&](const float* in, const float* w, const float* b, float* y) {
        hipLaunchKernelGGL(vt_layer_norm_kernel, dim3((unsigned)((M + 3) / 4)), dim3(kNT), 0, st,
                           in, w, b, y, M, D, dec.ln_eps);
        return hipGetLastError();
    };
    const int hd = (int)(D / dec.n_head);
    VT_TRY(ln(zhat, dec.ln1_weight, dec.ln1_bias, h));
    VT_TRY(gemm(h, dec.attn_weight, dec.attn_bias, qkv, D, 3 * D, nullptr, 0));
    if (dec.q_norm) {
        hipLaunchKernelGGL(vt_qk_norm_kernel, dim3((unsigned)M, 2 * dec.n_head), dim3(64), 0, st,
                           qkv, dec.q_norm, dec.k_norm, D, dec.n_head, hd, dec.qk_eps);
        VT_TRY(hipGetLastError());
    }
    hipLaunchKernelGGL(vt_attention_kernel, dim3((unsigned)L, dec.n_head, (unsigned)batch),
                       dim3(64), 0, st, qkv, a, L, D, hd, 1.0f / sqrtf((float)hd));
    VT_TRY(hipGetLastError());
    VT_TRY(gemm(a, dec.proj_weight, dec.proj_bias, x, D, D, zhat, 0));        // x = zhat + proj
    VT_TRY(ln(x, dec.ln2_weight, dec.ln2_bias, h));
    VT_TRY(gemm(h, dec.fc_weight, dec.fc_bias, f, D, 4 * D, nullptr, 1));     // GELU
    VT_TRY(gemm(f, dec.fc_proj_weight, dec.fc_proj_bias, x, 4 * D, D, x, 0)); // x += mlp
    VT_TRY(ln(x, dec.lnf_weight, nullptr, h));
    return gemm(h, dec.out_weight, nullptr, logits, D, C, nullptr, 0);
}

hipError_t vq_tok_reconstruct(const ncm_vq_tok_t& t, const int32_t* codes, int64_t batch,
                              float* zhat, void* ws, hipStream_t st) {
    Ws w;
    carve(t, batch, false, (char*)ws, &w);
    hipLaunchKernelGGL(vt_pad_rows_kernel, dim3(grid_for(batch * 2 * w.D)), dim3(kNT), 0, st,
                       w.hpad, batch, w.L, w.D);
    VT_TRY(hipGetLastError());
    int64_t off = 0;
    for (int l = 0; l < t.n_levels; ++l) {
        CodeSrc src{nullptr, codes, w.nsum, off, t.level_vocab[l]};
        VT_TRY(level_up(t, w, l, src, nullptr, st));
        VT_TRY(apply_resi(t, w, l, zhat, nullptr, st));
        off += t.level_len[l];
    }
    return hipSuccess;
}

}  // namespace ncm
