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
// reach a result. Calls on one GPU are ordered through one event per device
// (created with the address lookup): a call's stream waits for the event,
// then the call's kernels are queued and the event recorded after them, all
// under one host lock, so a call on another stream (or from another host
// thread) runs after the previous one. On a stream under graph capture the
// event is left out (a captured wait on an event recorded outside the
// capture is not portable): there the caller orders calls that share the
// array.
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
hipEvent_t g_scratch_done[kMaxDevices];  // the last call's kernels on that device

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
    hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p) {
        (void)hipGetLastError();
        ncm_set_error_detail(std::string("hipGetSymbolAddress(scratch): ") +
                             hipGetErrorString(e));
        return NCM_E_HIP;
    }
    hipEvent_t ev = nullptr;
    e = hipEventCreateWithFlags(&ev, hipEventDisableTiming);
    if (e != hipSuccess) {
        (void)hipGetLastError();
        ncm_set_error_detail(std::string("hipEventCreateWithFlags: ") + hipGetErrorString(e));
        return NCM_E_HIP;
    }
    g_scratch_done[device] = ev;
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
    // The lock covers the wait, the queued kernels and the record, so two
    // host threads cannot both queue work behind the same previous call.
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    void* ws = device >= 0 && device < kMaxDevices ? g_scratch_ptr[device] : nullptr;
    if (!ws) {
        ncm_set_error_detail("scratch address of this device was not looked up");
        return NCM_E_HIP;
    }
    const hipStream_t st = ncm_ctx_stream(ctx);
    hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
    hipError_t he = hipStreamIsCapturing(st, &cap);
    if (he != hipSuccess) {
        ncm_set_error_detail(std::string("hipStreamIsCapturing: ") + hipGetErrorString(he));
        return NCM_E_HIP;
    }
    const bool order = cap == hipStreamCaptureStatusNone;
    if (order && (he = hipStreamWaitEvent(st, g_scratch_done[device], 0)) != hipSuccess) {
        ncm_set_error_detail(std::string("hipStreamWaitEvent: ") + hipGetErrorString(he));
        return NCM_E_HIP;
    }
    rc = ncm::rvq_encode_ws(st, ws, (size_t)NCM_RVQ_SCRATCH_BYTES, x, b, t, d, levels, strides,
                            codebooks, csq, v, codes, recon, gap, force_codes, nullptr);
    // Recorded even after a failed call: whatever it queued is then ordered
    // before the next call.
    if (order && (he = hipEventRecord(g_scratch_done[device], st)) != hipSuccess) {
        ncm_set_error_detail(std::string("hipEventRecord: ") + hipGetErrorString(he));
        return rc ? rc : NCM_E_HIP;
    }
    return rc;
}
