// Host-side RVQ launchers and device-side argument blocks (internal).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/ncmorph_amd.h"

int ncm_ctx_workspace(ncm_ctx_t* ctx, size_t bytes, void** out);
hipStream_t ncm_ctx_stream(ncm_ctx_t* ctx);
int ncm_ctx_device(ncm_ctx_t* ctx);

namespace ncm {

// Looks up this device's address of the allocation-free encode's scratch
// array (once per device; the device must be current).
int noalloc_setup(int device);

constexpr int kMaxLevels = 32;
constexpr int kMaxPyr = 24;  // pyramid strides 2^1 .. 2^23
// Widest row the encode's row kernels hold: 16 chunks of 256 elements.
constexpr int64_t kMaxEncodeWidth = 4096;

struct LevelTable {
    int32_t stride[kMaxLevels];
    int64_t offset[kMaxLevels];  // code offset of each level inside a batch row
    int32_t levels;
    int64_t total;               // codes per batch row
};

// Everything a per-row RVQ kernel needs to locate its data.
struct RvqGeom {
    int64_t b, t, d, v;
    LevelTable L;
    int64_t pyr_off[kMaxPyr];  // float offset of the stride-2^j pool (j >= 1)
};

// Per-level counters of one encode: rows with an incomplete candidate chunk
// (every code of the chunk rescored) and rows that needed any exact
// distance (the others had one candidate under the threshold).
struct RvqCounts {
    int64_t levels;
    int64_t flagged[kMaxLevels];
    int64_t scored[kMaxLevels];
};

int rvq_check_shape(int64_t b, int64_t t, int64_t d, int64_t levels, const int32_t* strides,
                    int64_t v);
LevelTable make_level_table(int64_t t, int64_t levels, const int32_t* strides);

hipError_t launch_rvq_csq(const uint16_t* codebooks, int64_t rows, int64_t d, float* csq,
                          hipStream_t stream);
hipError_t launch_rvq_decode(const int32_t* codes, int64_t b, int64_t t, int64_t d,
                             int64_t levels, const int32_t* strides, const uint16_t* codebooks,
                             int64_t v, float* recon, hipStream_t stream);
int rvq_encode(ncm_ctx_t* ctx, const float* x, int64_t b, int64_t t, int64_t d, int64_t levels,
               const int32_t* strides, const uint16_t* codebooks, const float* csq, int64_t v,
               int32_t* codes, float* recon, float* gap, const int32_t* force_codes,
               int64_t* n_flagged, RvqCounts* counts = nullptr);
// Device bytes of the workspace one encode of this shape uses.
int rvq_workspace_bytes(int64_t b, int64_t t, int64_t d, int64_t levels, const int32_t* strides,
                        int64_t v, size_t* bytes);
// The encode on a caller-provided workspace (256-byte aligned, at least
// rvq_workspace_bytes long): allocates nothing.
int rvq_encode_ws(hipStream_t st, void* ws, size_t ws_bytes, const float* x, int64_t b,
                  int64_t t, int64_t d, int64_t levels, const int32_t* strides,
                  const uint16_t* codebooks, const float* csq, int64_t v, int32_t* codes,
                  float* recon, float* gap, const int32_t* force_codes, int64_t* n_flagged,
                  RvqCounts* counts = nullptr);

}  // namespace ncm
