// Host-side launchers of the HIP kernels (internal to the library).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace ncm {

// Tile configuration chosen for an M x N output (see the table in
// linear.hip); a valid `forced` index overrides the choice.
int linear_tile_config(int64_t M, int64_t N, int forced);

hipError_t launch_linear(const uint16_t* x, const uint16_t* w, const uint16_t* bias, void* y,
                         int64_t M, int64_t K, int64_t N, int out_mode, int config,
                         hipStream_t stream);

// fp32 operands, fp32 output; K % 4 == 0, 16-byte aligned x and w.
hipError_t launch_linear_f32(const float* x, const float* w, float* y, int64_t M, int64_t K,
                             int64_t N, hipStream_t stream);

// RMSNorm (bf16 mode, pinned cascade) of `rows` rows of width n; out_mode
// NCM_OUT_BF16_F32 (f32 holding bf16 values) or NCM_OUT_BF16 (bits).
hipError_t launch_rms_norm_rows(const float* x, const float* weight, void* y, int64_t rows,
                                int64_t n, float epsilon, int out_mode, hipStream_t stream);
// y = round_bf16(silu_bf16(gate) * up) (up NULL: silu_bf16(gate) alone).
hipError_t launch_silu_mul(const float* gate, const float* up, void* y, int64_t n, int out_mode,
                           hipStream_t stream);

hipError_t launch_bf16_from_f32(const float* src, uint16_t* dst, int64_t n, int flush,
                                hipStream_t stream);
// Row-padded variant: src [rows, cols] -> dst [rows, ld] (ld >= cols),
// columns [cols, ld) zero-filled.
hipError_t launch_bf16_from_f32_2d(const float* src, uint16_t* dst, int64_t rows, int64_t cols,
                                   int64_t ld, int flush, hipStream_t stream);
hipError_t launch_bf16_widen(const uint16_t* src, float* dst, int64_t n, hipStream_t stream);

}  // namespace ncm
