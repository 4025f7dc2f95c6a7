// Error detail and host-to-device upload shared by the host-side sources
// (definitions in api.hip, which owns the context).
#pragma once

#include <stddef.h>

#include <string>

#include "../../include/ncmorph_amd.h"

// Sets the text ncm_last_error() returns on this thread.
void ncm_set_error_detail(const std::string& what);

// Copies n host bytes to device memory on the context's stream through two
// pinned staging buffers; returns when the copies are enqueued and the host
// source is no longer read.
int ncm_upload_host_bytes(ncm_ctx_t* ctx, const void* src, void* dst, size_t n);
