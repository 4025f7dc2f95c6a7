// Shared device helpers for the gfx950 kernels: bf16 bit conversions,
// buffer resources and the wave-level vector types.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/ncmorph_amd.h"

namespace ncm {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));

constexpr int kWave = 64;

// RNE f32 -> bf16 bits, every NaN -> 0x7FC0, no flush
// (packages/bf16/root.zig:17-22).
__device__ __forceinline__ uint32_t bf16_bits_rne(float v) {
    uint32_t x = __float_as_uint(v);
    if ((x & 0x7FFFFFFFu) > 0x7F800000u) return 0x7FC0u;
    return (x + 0x7FFFu + ((x >> 16) & 1u)) >> 16;
}

// Round-to-nearest-even of two floats to bf16 in one v_cvt_pk_bf16_f32, a
// in the low half: the bits of bf16_bits_rne for every non-NaN input (a NaN
// becomes some quiet NaN instead of 0x7FC0).
__device__ __forceinline__ uint32_t bf16x2_rne(float a, float b) {
    const f32x2_t v = {a, b};
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2_t));
}

// bf16_bits_rne of a (low half) and b (high half), bit for bit, NaN -> 0x7FC0
// included: one v_cvt_pk_bf16_f32 and the NaN rule.
__device__ __forceinline__ uint32_t bf16x2_bits_rne(float a, float b) {
    uint32_t p = bf16x2_rne(a, b);
    p = a != a ? (p & 0xFFFF0000u) | 0x7FC0u : p;
    p = b != b ? (p & 0x0000FFFFu) | 0x7FC00000u : p;
    return p;
}

// Exponent bits zero -> signed zero (packages/kernels/root.zig:144-148).
__device__ __forceinline__ float flush_subnormal(float v) {
    uint32_t b = __float_as_uint(v);
    return (b & 0x7F800000u) == 0 ? __uint_as_float(b & 0x80000000u) : v;
}

// round(silu_bf16(gate) * up) of two elements from their accumulators
// (packages/kernels/root.zig:265-270, src/decoder.zig:210-211): the gate and
// up projections' bits (bf16(flush(acc + bias))), a = rb(g / (1 + expf(-g)))
// with rb(v) = v rounded to a bf16 value, then round(a * up); the roundings
// two values per v_cvt_pk_bf16_f32, bit for bit the same as bf16_bits_rne
// (the unfused SiLU x up kernel's arithmetic).
__device__ __forceinline__ void swiglu_bits2(float ga0, float ua0, float ga1, float ua1,
                                             float bg, float bu, uint32_t& o0, uint32_t& o1) {
    // Intermediate roundings without the NaN rule: a NaN stays a NaN through
    // the products and the quotient, and the final rounding maps it to 0x7FC0.
    const uint32_t p0 = bf16x2_rne(flush_subnormal(ga0 + bg), flush_subnormal(ua0 + bu));
    const uint32_t p1 = bf16x2_rne(flush_subnormal(ga1 + bg), flush_subnormal(ua1 + bu));
    const float g0 = __uint_as_float(p0 << 16), u0 = __uint_as_float(p0 & 0xFFFF0000u);
    const float g1 = __uint_as_float(p1 << 16), u1 = __uint_as_float(p1 & 0xFFFF0000u);
    const uint32_t a = bf16x2_rne(g0 / (1.0f + expf(-g0)), g1 / (1.0f + expf(-g1)));
    const uint32_t r = bf16x2_bits_rne(__uint_as_float(a << 16) * u0,
                                       __uint_as_float(a & 0xFFFF0000u) * u1);
    o0 = r & 0xFFFFu;
    o1 = r >> 16;
}

__device__ __forceinline__ float bf16_lo_to_f32(uint32_t packed) {
    return __uint_as_float(packed << 16);
}
__device__ __forceinline__ float bf16_hi_to_f32(uint32_t packed) {
    return __uint_as_float(packed & 0xFFFF0000u);
}

// Raw buffer resource over [base, base + bytes). Loads past `bytes` return
// zero, which is how partial tiles are zero-filled without branches.
// `base` and `bytes` must be wavefront-uniform; readfirstlane makes that
// explicit so the descriptor lives in SGPRs (a VGPR descriptor would force a
// waterfall loop around every load).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
    const uint64_t p = (uint64_t)base;
    const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)p);
    const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(p >> 32));
    const uint32_t n = __builtin_amdgcn_readfirstlane(bytes);
    void* up = (void*)(((uint64_t)hi << 32) | lo);
    return __builtin_amdgcn_make_buffer_rsrc(up, (short)0, (int)n, 0x00020000);
}

// An offset that is always outside any resource built above.
constexpr uint32_t kOobOffset = 0x80000000u;

__device__ __forceinline__ u32x4_t buffer_load_b128(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    return __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0);
}

// Workgroup barrier for LDS hand-off that leaves global loads in flight.
// __syncthreads() also waits for every outstanding vector-memory load
// (vmcnt(0)), which would drain the register prefetch of the next K tiles at
// each barrier. Here: wait for this wave's LDS operations (lgkmcnt(0)), then
// s_barrier; the empty asm statements keep the compiler from moving memory
// operations across the barrier.
__device__ __forceinline__ void lds_barrier() {
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0); vmcnt, expcnt unconstrained
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

// 4 x 4 transpose inside each quad of lanes (DPP quad permutes). Before:
// lane q of a quad holds M[j][q] in v[j]; after: lane q holds M[q][j].
// Applied to an MFMA D fragment (lane = column, element = row), it leaves
// each lane with four consecutive columns of one row.
__device__ __forceinline__ float dpp_quad_xor1(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0xB1, 0xF, 0xF, true));
}
__device__ __forceinline__ float dpp_quad_xor2(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x4E, 0xF, 0xF, true));
}
// Written as selects only (no conditional assignments), which compile to
// v_cndmask and DPP moves without branches.
__device__ __forceinline__ void quad_transpose4(float (&v)[4], int q) {
    const bool odd = (q & 1) != 0;
    const float r0 = dpp_quad_xor1(odd ? v[0] : v[1]);
    const float r1 = dpp_quad_xor1(odd ? v[2] : v[3]);
    const float a0 = odd ? r0 : v[0];
    const float a1 = odd ? v[1] : r0;
    const float a2 = odd ? r1 : v[2];
    const float a3 = odd ? v[3] : r1;
    const bool hi = (q & 2) != 0;
    const float u0 = dpp_quad_xor2(hi ? a0 : a2);
    const float u1 = dpp_quad_xor2(hi ? a1 : a3);
    v[0] = hi ? u0 : a0;
    v[1] = hi ? u1 : a1;
    v[2] = hi ? a2 : u0;
    v[3] = hi ? a3 : u1;
}

// Wavefront butterfly reductions in VALU (no LDS round trip): permlane32 /
// permlane16 swaps for the xor-32 and xor-16 stages, DPP for the others.
// Every stage combines the same two values as v op shfl_xor(v, off) does
// (after the xor-8 stage the values repeat with period 8 inside each row, so
// row_ror:4 meets the xor-4 partner's value), so for a commutative op the
// result has, in every lane, the bits of the xor butterfly with offsets
// 32, 16, 8, 4, 2, 1.
__device__ __forceinline__ u32x2_t swap32(uint32_t v) {
    auto r = __builtin_amdgcn_permlane32_swap(v, v, false, false);
    u32x2_t o; o[0] = r[0]; o[1] = r[1];
    return o;
}
__device__ __forceinline__ u32x2_t swap16(uint32_t v) {
    auto r = __builtin_amdgcn_permlane16_swap(v, v, false, false);
    u32x2_t o; o[0] = r[0]; o[1] = r[1];
    return o;
}
template <int CTRL>
__device__ __forceinline__ uint32_t dpp_u32(uint32_t v) {
    return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, 0xF, 0xF, false);
}
constexpr int kDppRor8 = 0x128, kDppRor4 = 0x124, kDppXor2 = 0x4E, kDppXor1 = 0xB1;

__device__ __forceinline__ float wave_sum_xor(float v) {
    u32x2_t p = swap32(__float_as_uint(v));
    v = __uint_as_float(p[0]) + __uint_as_float(p[1]);
    p = swap16(__float_as_uint(v));
    v = __uint_as_float(p[0]) + __uint_as_float(p[1]);
    v = v + __uint_as_float(dpp_u32<kDppRor8>(__float_as_uint(v)));
    v = v + __uint_as_float(dpp_u32<kDppRor4>(__float_as_uint(v)));
    v = v + __uint_as_float(dpp_u32<kDppXor2>(__float_as_uint(v)));
    v = v + __uint_as_float(dpp_u32<kDppXor1>(__float_as_uint(v)));
    return v;
}

__device__ __forceinline__ uint32_t wave_min_xor(uint32_t v) {
    u32x2_t p = swap32(v);
    v = min(p[0], p[1]);
    p = swap16(v);
    v = min(p[0], p[1]);
    v = min(v, dpp_u32<kDppRor8>(v));
    v = min(v, dpp_u32<kDppRor4>(v));
    v = min(v, dpp_u32<kDppXor2>(v));
    v = min(v, dpp_u32<kDppXor1>(v));
    return v;
}

__device__ __forceinline__ double wave_sum_xor_d(double v) {
    auto join = [](uint32_t lo, uint32_t hi) {
        return __longlong_as_double((long long)(((uint64_t)hi << 32) | lo));
    };
    auto lo = [](double x) { return (uint32_t)__double_as_longlong(x); };
    auto hi = [](double x) { return (uint32_t)((uint64_t)__double_as_longlong(x) >> 32); };
    u32x2_t pl = swap32(lo(v)), ph = swap32(hi(v));
    v = join(pl[0], ph[0]) + join(pl[1], ph[1]);
    pl = swap16(lo(v)); ph = swap16(hi(v));
    v = join(pl[0], ph[0]) + join(pl[1], ph[1]);
    v = v + join(dpp_u32<kDppRor8>(lo(v)), dpp_u32<kDppRor8>(hi(v)));
    v = v + join(dpp_u32<kDppRor4>(lo(v)), dpp_u32<kDppRor4>(hi(v)));
    v = v + join(dpp_u32<kDppXor2>(lo(v)), dpp_u32<kDppXor2>(hi(v)));
    v = v + join(dpp_u32<kDppXor1>(lo(v)), dpp_u32<kDppXor1>(hi(v)));
    return v;
}

// Remap a linear workgroup id so that consecutive logical tiles land on the
// same XCD (workgroups are dispatched round-robin over the 8 XCDs).
__device__ __forceinline__ int xcd_remap(int bid, int nblk) {
    constexpr int kXcd = 8;
    if (nblk % kXcd != 0) return bid;
    return (bid % kXcd) * (nblk / kXcd) + bid / kXcd;
}

}  // namespace ncm
