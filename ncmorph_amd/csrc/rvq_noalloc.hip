// Allocation-free multiscale RVQ encode: ncm_rvq_encode with its workspace
// in a fixed device array instead of the context's grow-only allocation, for
// callers that cannot allocate device memory (code under HIP graph capture,
// serving loops, harnesses that forbid hipMalloc).
//
// `scratch` is a file-scope device array of kRvqScratchBytes. Its host-side
// name is only a handle for the runtime: the device address of each GPU's
// copy comes from hipGetSymbolAddress, looked up once per device by
// ncm_init (with that device current) and kept in g_scratch_ptr. Kernels and
// host calls use that address, never the array's name.
//
// Every encode on one GPU shares that GPU's array, and the array keeps the
// previous call's contents. Each encode writes every workspace byte it reads
// (its set-up kernel zeroes the per-level counters), so stale contents never
// reach a result; two calls that overlap on one GPU (different streams, or
// different host threads) race on the array.
#include <hip/hip_runtime.h>

#include <mutex>
#include <string>

#include "../../include/ncmorph_amd.h"
#include "rvq.h"
#include "status.h"

static __device__ __align__(256) unsigned char scratch[NCM_RVQ_SCRATCH_BYTES];

namespace {

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices];

}  // namespace

namespace ncm {

int noalloc_setup(int device) {
    if (device < 0 || device >= kMaxDevices) {
        ncm_set_error_detail("device index beyond the scratch table");
        return NCM_E_DEVICE;
    }
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (g_scratch_ptr[device]) return NCM_OK;
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p) {
        (void)hipGetLastError();
        ncm_set_error_detail(std::string("hipGetSymbolAddress(scratch): ") +
                             hipGetErrorString(e));
        return NCM_E_HIP;
    }
    g_scratch_ptr[device] = p;
    return NCM_OK;
}

}  // namespace ncm

extern "C" int ncm_rvq_encode_noalloc(ncm_ctx_t* ctx, const float* x, int64_t b, int64_t t,
                                      int64_t d, int64_t levels, const int32_t* strides,
                                      const uint16_t* codebooks, const float* csq, int64_t v,
                                      int32_t* codes, float* recon, float* gap,
                                      const int32_t* force_codes) {
    if (!ctx) return NCM_E_NULL;
    if (!x || !strides || !codebooks || !csq || !codes) return NCM_E_NULL;
    int rc = ncm::rvq_check_shape(b, t, d, levels, strides, v);
    if (rc) return rc;
    size_t bytes = 0;
    rc = ncm::rvq_workspace_bytes(b, t, d, levels, strides, v, &bytes);
    if (rc) return rc;
    if (bytes > (size_t)NCM_RVQ_SCRATCH_BYTES) {
        ncm_set_error_detail("encode needs " + std::to_string(bytes) +
                             " workspace bytes; the fixed scratch holds " +
                             std::to_string((size_t)NCM_RVQ_SCRATCH_BYTES));
        return NCM_E_SCRATCH;
    }
    const int device = ncm_ctx_device(ctx);
    const hipError_t e = hipSetDevice(device);
    if (e != hipSuccess) {
        ncm_set_error_detail(std::string("hipSetDevice: ") + hipGetErrorString(e));
        return NCM_E_HIP;
    }
    void* ws = nullptr;
    {
        std::lock_guard<std::mutex> lock(g_scratch_mu);
        if (device >= 0 && device < kMaxDevices) ws = g_scratch_ptr[device];
    }
    if (!ws) {
        ncm_set_error_detail("scratch address of this device was not looked up");
        return NCM_E_HIP;
    }
    return ncm::rvq_encode_ws(ncm_ctx_stream(ctx), ws, (size_t)NCM_RVQ_SCRATCH_BYTES, x, b, t, d,
                              levels, strides, codebooks, csq, v, codes, recon, gap, force_codes,
                              nullptr);
}
