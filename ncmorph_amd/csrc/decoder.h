// Decoder prefill forward (internal; the C entry point is in api.hip).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/ncmorph_amd.h"

namespace ncm {

size_t decoder_workspace_bytes(const ncm_decoder_shape_t& s, int64_t batch, int64_t seq);

// All pointers device memory except `layers` (host array) and `host_ids`.
hipError_t decoder_forward(const ncm_decoder_shape_t& s, const ncm_decoder_layer_t* layers,
                           const uint16_t* embed, const float* final_norm,
                           const uint16_t* lm_head, const float* cosine, const float* sine,
                           const int64_t* host_ids, int64_t batch, int64_t seq, float* logits,
                           void* ws, hipStream_t st);

}  // namespace ncm
