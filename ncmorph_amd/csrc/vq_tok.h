// Host-side launchers of the VQ-VAE tokenizer kernels (vq_tok.hip,
// vq_tok_decoder.hip); internal to the library.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/ncmorph_amd.h"

namespace ncm {

// Workspace of vq_tok_encode / vq_tok_reconstruct for `batch` sequences
// (need_zhat: room for the reconstruction when the caller keeps none).
size_t vq_tok_workspace_bytes(const ncm_vq_tok_t& t, int64_t batch, bool need_zhat);

hipError_t vq_tok_pack_conv(const float* src, float* dst, int64_t c, int64_t k, int transposed,
                            hipStream_t st);

// ids_host (int32, [batch, L], validated) or latent_in (device [batch, L, D]).
hipError_t vq_tok_encode(const ncm_vq_tok_t& t, const int32_t* ids_host, const float* latent_in,
                         int64_t batch, int32_t* codes, float* zhat, float* latent_out, void* ws,
                         hipStream_t st);

hipError_t vq_tok_reconstruct(const ncm_vq_tok_t& t, const int32_t* codes, int64_t batch,
                              float* zhat, void* ws, hipStream_t st);

// The decoder block, ln_f and the output layer on zhat [batch, L, D] ->
// logits [batch, L, C].
size_t vq_tok_decoder_workspace_bytes(const ncm_vq_tok_t& t, int64_t batch);
hipError_t vq_tok_decode(const ncm_vq_tok_t& t, const ncm_vq_tok_decoder_t& dec, const float* zhat,
                         int64_t batch, float* logits, void* ws, hipStream_t st);

}  // namespace ncm
