// NCM level-parallel body (internal; the C entry point is in api.hip).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/ncmorph_amd.h"

namespace ncm {

constexpr int kMaxNcmLevels = NCM_MAX_LEVELS;

size_t ncm_workspace_bytes(const ncm_ncm_shape_t& s, bool convs);

// All pointers device memory except `layers` and the conv pointer arrays of
// `w` (host arrays), host_ids [prefix_length] and host_pad [pad_len].
// hidden_states: null or float [layers + 1, S, hidden] (the reference's
// forward_with_trace states).
hipError_t ncm_forward(const ncm_ncm_shape_t& s, const ncm_decoder_layer_t* layers,
                       const ncm_ncm_weights_t& w, const int64_t* host_ids,
                       const uint8_t* host_pad, int64_t pad_len, const float* target,
                       const float* cosine, const float* sine, float* output,
                       float* hidden_states, void* ws, hipStream_t st);

// The same body in the reference's f32 arithmetic (float weights,
// ncm_decoder_layer_f32_t layers); same pointer conventions.
size_t ncm_f32_workspace_bytes(const ncm_ncm_shape_t& s, bool convs);
hipError_t ncm_forward_f32(const ncm_ncm_shape_t& s, const ncm_decoder_layer_f32_t* layers,
                           const ncm_ncm_weights_f32_t& w, const int64_t* host_ids,
                           const uint8_t* host_pad, int64_t pad_len, const float* target,
                           const float* cosine, const float* sine, float* output,
                           float* hidden_states, void* ws, hipStream_t st);

}  // namespace ncm
