// C ABI of ncmorph_amd (include/ncmorph_amd.h): contexts, argument checks,
// the host-slice drop-ins for the reference's Zig kernels, and the
// device-resident entry points.
#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstring>
#include <condition_variable>
#include <mutex>
#include <string>
#include <thread>
#include <vector>
#include <algorithm>

#include "../../include/ncmorph_amd.h"
#include "decoder.h"
#include "linear.h"
#include "ncm_body.h"
#include "rvq.h"
#include "status.h"
#include "vq_tok.h"

struct ncm_ctx {
    int device = 0;
    hipStream_t own_stream = nullptr;
    hipStream_t stream = nullptr;
    void* ws = nullptr;  // grow-only device workspace
    size_t ws_bytes = 0;
    hipEvent_t handoff = nullptr;  // orders a new stream after the previous one
    // Pinned staging of host -> device uploads (two buffers of stage_bytes,
    // each with the event of its last copy), kept until ncm_destroy.
    void* stage[2] = {nullptr, nullptr};
    hipEvent_t stage_done[2] = {nullptr, nullptr};
    size_t stage_bytes = 0;
};

namespace {

thread_local std::string g_last_error;

int fail_hip(hipError_t e, const char* what) {
    g_last_error = std::string(what) + ": " + hipGetErrorString(e);
    return NCM_E_HIP;
}

#define NCM_HIP(call)                                        \
    do {                                                     \
        hipError_t e_ = (call);                              \
        if (e_ != hipSuccess) return fail_hip(e_, #call);    \
    } while (0)

bool is_gfx950(int device) {
    hipDeviceProp_t p;
    if (hipGetDeviceProperties(&p, device) != hipSuccess) return false;
    return std::strncmp(p.gcnArchName, "gfx950", 6) == 0;
}

int ctx_bind(ncm_ctx_t* ctx) {
    NCM_HIP(hipSetDevice(ctx->device));
    return NCM_OK;
}

}  // namespace

// Grow-only workspace. Growing waits for the stream so the old buffer is no
// longer in use before it is released.
int ncm_ctx_workspace(ncm_ctx_t* ctx, size_t bytes, void** out) {
    if (bytes > ctx->ws_bytes) {
        if (ctx->ws) {
            NCM_HIP(hipStreamSynchronize(ctx->stream));
            NCM_HIP(hipFree(ctx->ws));
            ctx->ws = nullptr;
            ctx->ws_bytes = 0;
        }
        size_t want = bytes + (bytes >> 3);
        hipError_t e = hipMalloc(&ctx->ws, want);
        if (e != hipSuccess) {
            (void)hipGetLastError();
            ctx->ws = nullptr;
            g_last_error = std::string("hipMalloc workspace: ") + hipGetErrorString(e);
            return NCM_E_NOMEM;
        }
        ctx->ws_bytes = want;
    }
    *out = ctx->ws;
    return NCM_OK;
}

hipStream_t ncm_ctx_stream(ncm_ctx_t* ctx) { return ctx->stream; }

int ncm_ctx_device(ncm_ctx_t* ctx) { return ctx->device; }

void ncm_set_error_detail(const std::string& what) { g_last_error = what; }

// memcpy of one buffer by a pool of threads (one thread moves ~10-15 GB/s
// from the page cache; the host link takes several times that): the caller
// copies the first slice, the workers the others.
class CopyPool {
  public:
    explicit CopyPool(int threads) : n_(threads < 1 ? 1 : threads) {
        // A thread that cannot be started leaves its slices to the others
        // (n_ counts the threads that run, the caller included).
        int started = 1;
        try {
            for (int t = 1; t < n_; ++t) {
                th_.emplace_back([this, t] { work(t); });
                ++started;
            }
        } catch (...) {
        }
        n_ = started;
    }
    ~CopyPool() {
        {
            std::lock_guard<std::mutex> lk(mu_);
            stop_ = true;
        }
        go_.notify_all();
        for (auto& t : th_) t.join();
    }
    void copy(char* to, const char* from, size_t len) {
        const size_t slice = (len + n_ - 1) / n_;
        {
            std::lock_guard<std::mutex> lk(mu_);
            to_ = to; from_ = from; len_ = len; slice_ = slice;
            pending_ = n_ - 1;
            ++gen_;
        }
        go_.notify_all();
        std::memcpy(to, from, std::min(len, slice));
        std::unique_lock<std::mutex> lk(mu_);
        done_.wait(lk, [this] { return pending_ == 0; });
    }

  private:
    void work(int t) {
        uint64_t seen = 0;
        std::unique_lock<std::mutex> lk(mu_);
        for (;;) {
            go_.wait(lk, [&] { return stop_ || gen_ != seen; });
            if (stop_) return;
            seen = gen_;
            char* to = to_;
            const char* from = from_;
            const size_t a = (size_t)t * slice_, len = len_;
            lk.unlock();
            if (a < len) std::memcpy(to + a, from + a, std::min(len, a + slice_) - a);
            lk.lock();
            if (--pending_ == 0) done_.notify_one();
        }
    }
    int n_;
    std::vector<std::thread> th_;
    std::mutex mu_;
    std::condition_variable go_, done_;
    char* to_ = nullptr;
    const char* from_ = nullptr;
    size_t len_ = 0, slice_ = 0;
    uint64_t gen_ = 0;
    int pending_ = 0;
    bool stop_ = false;
};

int ncm_upload_host_bytes(ncm_ctx_t* ctx, const void* src, void* dst, size_t n) {
    int rc = ctx_bind(ctx);
    if (rc) return rc;
    // The context's two pinned staging buffers, refilled from the (mapped,
    // pageable) source while the other one's copy runs; allocated when an
    // upload needs more than they hold (at least doubling, at most 64 MiB
    // each) and kept, since pinning memory costs milliseconds per call.
    constexpr size_t kChunk = 64u << 20;
    const size_t chunk = n < kChunk ? n : kChunk;
    if (ctx->stage_bytes < chunk) {
        const size_t want = std::max(chunk, std::min(kChunk, 2 * ctx->stage_bytes));
        for (int b = 0; b < 2; ++b) {
            if (ctx->stage_done[b]) (void)hipEventSynchronize(ctx->stage_done[b]);
            if (ctx->stage[b]) (void)hipHostFree(ctx->stage[b]);
            ctx->stage[b] = nullptr;
        }
        ctx->stage_bytes = 0;
        for (int b = 0; b < 2; ++b) {
            if (hipHostMalloc(&ctx->stage[b], want, hipHostMallocDefault) != hipSuccess) {
                (void)hipGetLastError();
                for (int c = 0; c < 2; ++c) {
                    if (ctx->stage[c]) (void)hipHostFree(ctx->stage[c]);
                    ctx->stage[c] = nullptr;
                }
                g_last_error = "pinned staging allocation failed";
                return NCM_E_NOMEM;
            }
        }
        ctx->stage_bytes = want;
    }
    for (int b = 0; b < 2; ++b)
        if (!ctx->stage_done[b])
            NCM_HIP(hipEventCreateWithFlags(&ctx->stage_done[b], hipEventDisableTiming));
    // At most 16 copy threads (the host's share for one GPU), fewer on a
    // smaller host, one for small uploads.
    const unsigned hw = std::thread::hardware_concurrency();
    const int threads = n < (4u << 20) ? 1 : (int)std::min<unsigned>(16u, hw ? hw : 1u);
    CopyPool pool(threads);
    size_t off = 0;
    for (int b = 0; off < n; b ^= 1) {
        const size_t len = n - off < chunk ? n - off : chunk;
        hipError_t e = hipEventSynchronize(ctx->stage_done[b]);  // the buffer's last copy is done
        if (e == hipSuccess) {
            pool.copy((char*)ctx->stage[b], (const char*)src + off, len);
            e = hipMemcpyAsync((char*)dst + off, ctx->stage[b], len, hipMemcpyHostToDevice,
                               ctx->stream);
        }
        if (e == hipSuccess) e = hipEventRecord(ctx->stage_done[b], ctx->stream);
        if (e != hipSuccess) return fail_hip(e, "upload");
        off += len;
    }
    // The device holds the bytes when the call returns.
    for (int b = 0; b < 2; ++b) NCM_HIP(hipEventSynchronize(ctx->stage_done[b]));
    return NCM_OK;
}

extern "C" {

const char* ncm_status_string(int status) {
    switch (status) {
        case NCM_OK: return "ok";
        case NCM_E_NULL: return "null pointer argument";
        case NCM_E_SHAPE: return "invalid or unsupported shape";
        case NCM_E_LENGTH: return "slice length does not match dimensions";
        case NCM_E_HIP: return "HIP runtime error";
        case NCM_E_NOMEM: return "allocation failed";
        case NCM_E_DEVICE: return "no usable gfx950 device";
        case NCM_E_ARG: return "argument out of range";
        case NCM_E_FORMAT: return "malformed file or header";
        case NCM_E_SCRATCH: return "shape exceeds the fixed scratch buffer";
        default: return "unknown status";
    }
}

const char* ncm_last_error(void) { return g_last_error.c_str(); }

int ncm_init(int device, ncm_ctx_t** out) {
    if (!out) return NCM_E_NULL;
    *out = nullptr;
    int count = 0;
    if (hipGetDeviceCount(&count) != hipSuccess || device < 0 || device >= count) {
        (void)hipGetLastError();
        g_last_error = "no HIP device with this index";
        return NCM_E_DEVICE;
    }
    if (!is_gfx950(device)) {
        g_last_error = "device is not gfx950";
        return NCM_E_DEVICE;
    }
    ncm_ctx_t* ctx = new ncm_ctx();
    ctx->device = device;
    hipError_t e = hipSetDevice(device);
    if (e == hipSuccess) e = hipStreamCreateWithFlags(&ctx->own_stream, hipStreamNonBlocking);
    if (e != hipSuccess) {
        delete ctx;
        return fail_hip(e, "ncm_init");
    }
    ctx->stream = ctx->own_stream;
    // The allocation-free entry points need this device's scratch address.
    const int rc = ncm::noalloc_setup(device);
    if (rc) {
        (void)hipStreamDestroy(ctx->own_stream);
        delete ctx;
        return rc;
    }
    *out = ctx;
    return NCM_OK;
}

int ncm_destroy(ncm_ctx_t* ctx) {
    if (!ctx) return NCM_E_NULL;
    (void)hipSetDevice(ctx->device);
    if (ctx->stream) (void)hipStreamSynchronize(ctx->stream);
    if (ctx->ws) (void)hipFree(ctx->ws);
    if (ctx->handoff) (void)hipEventDestroy(ctx->handoff);
    for (int b = 0; b < 2; ++b) {
        if (ctx->stage_done[b]) {
            (void)hipEventSynchronize(ctx->stage_done[b]);
            (void)hipEventDestroy(ctx->stage_done[b]);
        }
        if (ctx->stage[b]) (void)hipHostFree(ctx->stage[b]);
    }
    if (ctx->own_stream) (void)hipStreamDestroy(ctx->own_stream);
    delete ctx;
    return NCM_OK;
}

int ncm_set_stream(ncm_ctx_t* ctx, void* stream) {
    if (!ctx) return NCM_E_NULL;
    // NULL selects HIP's default (null) stream, as everywhere in HIP.
    hipStream_t next = (hipStream_t)stream;
    if (next != ctx->stream && ctx->ws) {
        // Every entry point shares the one workspace: work queued on the new
        // stream waits for everything already queued on the previous one, so
        // two streams never use the workspace at the same time.
        int rc = ctx_bind(ctx);
        if (rc) return rc;
        if (!ctx->handoff)
            NCM_HIP(hipEventCreateWithFlags(&ctx->handoff, hipEventDisableTiming));
        NCM_HIP(hipEventRecord(ctx->handoff, ctx->stream));
        NCM_HIP(hipStreamWaitEvent(next, ctx->handoff, 0));
    }
    ctx->stream = next;
    return NCM_OK;
}

void* ncm_get_stream(ncm_ctx_t* ctx) { return ctx ? (void*)ctx->stream : nullptr; }

int ncm_synchronize(ncm_ctx_t* ctx) {
    if (!ctx) return NCM_E_NULL;
    int rc = ctx_bind(ctx);
    if (rc) return rc;
    NCM_HIP(hipStreamSynchronize(ctx->stream));
    return NCM_OK;
}

// ------------------------------------------------------------------ linear

int ncm_linear_bf16(ncm_ctx_t* ctx, const uint16_t* x, const uint16_t* w, const uint16_t* bias,
                    void* y, int64_t m, int64_t k, int64_t n, int out_mode) {
    if (!ctx) return NCM_E_NULL;
    if (m < 0 || n < 0 || k < 0) return NCM_E_SHAPE;
    if (out_mode < NCM_OUT_F32 || out_mode > NCM_OUT_BF16) return NCM_E_ARG;
    if (m == 0 || n == 0) return NCM_OK;
    if (!y || (k > 0 && (!x || !w))) return NCM_E_NULL;
    // Rows must be 16-byte aligned for the vector loads; the loader's byte
    // offsets must fit 31 bits inside one tile.
    if (k % 8 != 0 || k > (int64_t(1) << 21)) return NCM_E_SHAPE;
    if ((uintptr_t)x % 16 || (uintptr_t)w % 16) return NCM_E_ARG;
    if (m > (int64_t(1) << 31) || n > (int64_t(1) << 31)) return NCM_E_SHAPE;
    int rc = ctx_bind(ctx);
    if (rc) return rc;
    hipError_t e = ncm::launch_linear(x, w, bias, y, m, k, n, out_mode, -1, ctx->stream);
    if (e != hipSuccess) return fail_hip(e, "linear kernel launch");
    return NCM_OK;
}

int ncm_linear_bf16_exact(ncm_ctx_t* ctx, const uint16_t* x, const uint16_t* w,
                          const uint16_t* bias, void* y, int64_t m, int64_t k, int64_t n,
                          int out_mode) {
    if (!ctx) return NCM_E_NULL;
    if (m < 0 || n < 0 || k < 0) return NCM_E_SHAPE;
    if (out_mode < NCM_OUT_F32 || out_mode > NCM_OUT_BF16) return NCM_E_ARG;
    if (m == 0 || n == 0) return NCM_OK;
    if (!y || (k > 0 && (!x || !w))) return NCM_E_NULL;
    if (m > (int64_t(1) << 31) || n > (int64_t(1) << 31) || k > (int64_t(1) << 31) ||
        ((m + 63) / 64) * ((n + 63) / 64) > 0x7FFFFFFF)
        return NCM_E_SHAPE;
    int rc = ctx_bind(ctx);
    if (rc) return rc;
    hipError_t e = ncm::launch_linear_exact(x, w, bias, y, m, k, n, out_mode, ctx->stream);
    if (e != hipSuccess) return fail_hip(e, "exact linear kernel launch");
    return NCM_OK;
}

int ncm_linear_bf16_residual(ncm_ctx_t* ctx, const uint16_t* x, const uint16_t* w,
                             const uint16_t* bias, const float* residual, void* y, int64_t m,
                             int64_t k, int64_t n, int out_mode) {
    if (!ctx) return NCM_E_NULL;
    if (m < 0 || n < 0 || k < 0) return NCM_E_SHAPE;
    if (out_mode < NCM_OUT_F32 || out_mode > NCM_OUT_BF16) return NCM_E_ARG;
    if (m == 0 || n == 0) return NCM_OK;
    if (!y || !residual || (k > 0 && (!x || !w))) return NCM_E_NULL;
    if (k % 8 != 0 || k > (int64_t(1) << 21)) return NCM_E_SHAPE;
    if ((uintptr_t)x % 16 || (uintptr_t)w % 16) return NCM_E_ARG;
    // In place only where y holds fp32 values at the residual's addresses.
    if (out_mode == NCM_OUT_BF16 && (const void*)residual == y) return NCM_E_ARG;
    if (m > (int64_t(1) << 31) || n > (int64_t(1) << 31)) return NCM_E_SHAPE;
    int rc = ctx_bind(ctx);
    if (rc) return rc;
    hipError_t e = ncm::launch_linear_residual(x, w, bias, residual, y, m, k, n, out_mode,
                                               ctx->stream);
    if (e != hipSuccess) return fail_hip(e, "residual linear kernel launch");
    return NCM_OK;
}

namespace {
int check_linear_args(const void* x, const void* w, const void* y, int64_t m, int64_t k,
                      int64_t n) {
    if (m < 0 || n < 0 || k < 0) return NCM_E_SHAPE;
    if (m == 0 || n == 0) return NCM_OK;
    if (!y || (k > 0 && (!x || !w))) return NCM_E_NULL;
    if (k % 8 != 0 || k > (int64_t(1) << 21)) return NCM_E_SHAPE;
    if ((uintptr_t)x % 16 || (uintptr_t)w % 16 || (uintptr_t)y % 8) return NCM_E_ARG;
    if (m > (int64_t(1) << 31) || n > (int64_t(1) << 31)) return NCM_E_SHAPE;
    return NCM_OK;
}
}  // namespace

int ncm_linear_bf16_swiglu(ncm_ctx_t* ctx, const uint16_t* x, const uint16_t* w,
                           const uint16_t* bias, uint16_t* y, int64_t m, int64_t k,
                           int64_t n2) {
    if (!ctx) return NCM_E_NULL;
    int rc = check_linear_args(x, w, y, m, k, n2);
    if (rc) return rc;
    if (n2 % 64) return NCM_E_SHAPE;
    if (m == 0 || n2 == 0) return NCM_OK;
    rc = ctx_bind(ctx);
    if (rc) return rc;
    hipError_t e = ncm::launch_linear_swiglu(x, w, bias, y, m, k, n2, ctx->stream);
    if (e != hipSuccess) return fail_hip(e, "swiglu linear launch");
    return NCM_OK;
}

int ncm_linear_bf16_rope64(ncm_ctx_t* ctx, const uint16_t* x, const uint16_t* w,
                           const uint16_t* bias, uint16_t* y, int64_t m, int64_t k, int64_t n,
                           int64_t rot_cols, int64_t seq_len, const float* cosine,
                           const float* sine) {
    if (!ctx) return NCM_E_NULL;
    int rc = check_linear_args(x, w, y, m, k, n);
    if (rc) return rc;
    if (n % 64 || rot_cols < 0 || rot_cols % 64 || rot_cols > n || seq_len <= 0)
        return NCM_E_SHAPE;
    if (m == 0 || n == 0) return NCM_OK;
    if (rot_cols > 0 && (!cosine || !sine)) return NCM_E_NULL;
    rc = ctx_bind(ctx);
    if (rc) return rc;
    hipError_t e = ncm::launch_linear_rope64(x, w, bias, y, m, k, n, rot_cols, seq_len, cosine,
                                             sine, ctx->stream);
    if (e != hipSuccess) return fail_hip(e, "rope linear launch");
    return NCM_OK;
}

int ncm_tied_head_logits_levels(ncm_ctx_t* ctx, const uint16_t* z, const uint16_t* codebooks,
                                const float* csq, const float* bias, const float* log_inv_t,
                                const int64_t* level_rows, int64_t n_levels, int64_t d,
                                int64_t v, float* logits) {
    if (!ctx) return NCM_E_NULL;
    if (n_levels < 1 || n_levels > 32 || v < 1) return NCM_E_SHAPE;
    if (!log_inv_t || !level_rows) return NCM_E_NULL;
    int64_t rows = 0;
    for (int64_t l = 0; l < n_levels; ++l) {
        if (level_rows[l] < 0) return NCM_E_SHAPE;
        rows += level_rows[l];
        if (rows > (int64_t(1) << 31)) return NCM_E_SHAPE;
    }
    int rc = check_linear_args(z, codebooks, logits, rows, d, v);
    if (rc) return rc;
    if (!csq) return NCM_E_NULL;
    if (rows == 0) return NCM_OK;
    rc = ctx_bind(ctx);
    if (rc) return rc;
    void* ws = nullptr;
    rc = ncm_ctx_workspace(ctx, 256, &ws);
    if (rc) return rc;
    hipError_t e = ncm::launch_tied_head(z, codebooks, csq, bias, log_inv_t, level_rows,
                                         (int)n_levels, (float*)ws, logits, d, v, ctx->stream);
    if (e == hipErrorInvalidConfiguration) return NCM_E_SHAPE;
    if (e != hipSuccess) return fail_hip(e, "tied head launch");
    return NCM_OK;
}

int ncm_tied_head_logits(ncm_ctx_t* ctx, const uint16_t* z, const uint16_t* codebook,
                         const float* csq, const float* bias, float log_inv_t, float* logits,
                         int64_t rows, int64_t d, int64_t v) {
    if (rows < 0) return NCM_E_SHAPE;
    return ncm_tied_head_logits_levels(ctx, z, codebook, csq, bias, &log_inv_t, &rows, 1, d, v,
                                       logits);
}

int ncm_linear_f32(ncm_ctx_t* ctx, const float* x, const float* w, float* y, int64_t m,
                   int64_t k, int64_t n) {
    if (!ctx) return NCM_E_NULL;
    if (m < 0 || n < 0 || k < 0) return NCM_E_SHAPE;
    if (m == 0 || n == 0) return NCM_OK;
    if (!y || (k > 0 && (!x || !w))) return NCM_E_NULL;
    if (k % 4 != 0 || k > (int64_t(1) << 20)) return NCM_E_SHAPE;
    if ((uintptr_t)x % 16 || (uintptr_t)w % 16) return NCM_E_ARG;
    if (m > (int64_t(1) << 31) || n > (int64_t(1) << 31)) return NCM_E_SHAPE;
    int rc = ctx_bind(ctx);
    if (rc) return rc;
    hipError_t e = ncm::launch_linear_f32(x, w, y, m, k, n, ctx->stream);
    if (e != hipSuccess) return fail_hip(e, "f32 linear kernel launch");
    return NCM_OK;
}

int ncm_bf16_from_f32_dev(ncm_ctx_t* ctx, const float* src, uint16_t* dst, int64_t n,
                          int flush) {
    if (!ctx) return NCM_E_NULL;
    if (n < 0) return NCM_E_SHAPE;
    if (n == 0) return NCM_OK;
    if (!src || !dst) return NCM_E_NULL;
    int rc = ctx_bind(ctx);
    if (rc) return rc;
    hipError_t e = ncm::launch_bf16_from_f32(src, dst, n, flush ? 1 : 0, ctx->stream);
    if (e != hipSuccess) return fail_hip(e, "bf16 conversion launch");
    return NCM_OK;
}

int ncm_bf16_widen_dev(ncm_ctx_t* ctx, const uint16_t* src, float* dst, int64_t n) {
    if (!ctx) return NCM_E_NULL;
    if (n < 0) return NCM_E_SHAPE;
    if (n == 0) return NCM_OK;
    if (!src || !dst) return NCM_E_NULL;
    int rc = ctx_bind(ctx);
    if (rc) return rc;
    hipError_t e = ncm::launch_bf16_widen(src, dst, n, ctx->stream);
    if (e != hipSuccess) return fail_hip(e, "bf16 widen launch");
    return NCM_OK;
}

// ------------------------------------------------------------------ decoder ops

int ncm_rms_norm_rows_dev(ncm_ctx_t* ctx, const float* x, const float* weight, void* y,
                          int64_t rows, int64_t width, float epsilon, int out_mode) {
    if (!ctx) return NCM_E_NULL;
    if (rows < 0 || width < 0) return NCM_E_SHAPE;
    if (out_mode != NCM_OUT_F32 && out_mode != NCM_OUT_BF16_F32 && out_mode != NCM_OUT_BF16)
        return NCM_E_ARG;
    if (rows == 0) return NCM_OK;
    if (width == 0) return NCM_E_SHAPE;  // root.zig:247: nonempty rows
    if (!x || !weight || !y) return NCM_E_NULL;
    if (width % 4 == 0 && ((uintptr_t)x % 16 || (uintptr_t)weight % 16)) return NCM_E_ARG;
    int rc = ctx_bind(ctx);
    if (rc) return rc;
    hipError_t e = ncm::launch_rms_norm_rows(x, weight, y, rows, width, epsilon, out_mode,
                                             ctx->stream);
    if (e != hipSuccess) return fail_hip(e, "rms_norm launch");
    return NCM_OK;
}

int ncm_silu_mul_dev(ncm_ctx_t* ctx, const float* gate, const float* up, void* y, int64_t n,
                     int out_mode) {
    if (!ctx) return NCM_E_NULL;
    if (n < 0) return NCM_E_SHAPE;
    if (out_mode != NCM_OUT_F32 && out_mode != NCM_OUT_BF16_F32 && out_mode != NCM_OUT_BF16)
        return NCM_E_ARG;
    if (n == 0) return NCM_OK;
    if (!gate || !y) return NCM_E_NULL;
    int rc = ctx_bind(ctx);
    if (rc) return rc;
    hipError_t e = ncm::launch_silu_mul(gate, up, y, n, out_mode, ctx->stream);
    if (e != hipSuccess) return fail_hip(e, "silu_mul launch");
    return NCM_OK;
}

int ncm_rope_rotate_dev(ncm_ctx_t* ctx, uint16_t* x, int64_t rows, int64_t row_stride,
                        int heads, int head_dim, int64_t seq_len, const float* cosine,
                        const float* sine) {
    if (!ctx) return NCM_E_NULL;
    if (rows < 0 || heads < 0 || head_dim <= 0 || head_dim % 2 || seq_len <= 0)
        return NCM_E_SHAPE;
    if (row_stride < (int64_t)heads * head_dim) return NCM_E_SHAPE;
    if (rows == 0 || heads == 0) return NCM_OK;
    if (!x || !cosine || !sine) return NCM_E_NULL;
    if (rows > (int64_t(1) << 40) || (int64_t)heads * head_dim > (int64_t(1) << 31) ||
        rows * heads * (int64_t)(head_dim / 2) > (int64_t(1) << 40))
        return NCM_E_SHAPE;
    int rc = ctx_bind(ctx);
    if (rc) return rc;
    hipError_t e = ncm::launch_rope_rotate(x, rows, row_stride, heads, head_dim, seq_len, cosine,
                                           sine, ctx->stream);
    if (e != hipSuccess) return fail_hip(e, "rope rotate launch");
    return NCM_OK;
}

int ncm_attention_bf16_dev(ncm_ctx_t* ctx, const uint16_t* q, const uint16_t* k,
                           const uint16_t* v, void* out, int64_t batch, int64_t seq_len,
                           int q_heads, int kv_heads, int head_dim, int64_t q_stride,
                           int64_t kv_stride, int64_t out_stride, int64_t window, int out_mode) {
    if (!ctx) return NCM_E_NULL;
    if (batch < 0 || seq_len < 0 || q_heads <= 0 || kv_heads <= 0 || window < 0)
        return NCM_E_SHAPE;
    if (head_dim != 64 && head_dim != 128) return NCM_E_SHAPE;
    if (q_heads % kv_heads) return NCM_E_SHAPE;
    if (out_mode != NCM_OUT_BF16_F32 && out_mode != NCM_OUT_BF16) return NCM_E_ARG;
    if (q_stride < (int64_t)q_heads * head_dim || kv_stride < (int64_t)kv_heads * head_dim ||
        out_stride < (int64_t)q_heads * head_dim)
        return NCM_E_SHAPE;
    if (batch == 0 || seq_len == 0) return NCM_OK;
    if (!q || !k || !v || !out) return NCM_E_NULL;
    // 16-byte row segments for the vector loads.
    if (q_stride % 8 || kv_stride % 8) return NCM_E_ARG;
    if ((uintptr_t)q % 16 || (uintptr_t)k % 16 || (uintptr_t)v % 16) return NCM_E_ARG;
    if (batch > 65535 || q_heads > 65535 || seq_len > (int64_t(1) << 31)) return NCM_E_SHAPE;
    int rc = ctx_bind(ctx);
    if (rc) return rc;
    void* vt = nullptr;
    rc = ncm_ctx_workspace(ctx, ncm::attention_workspace_bytes(batch, seq_len, kv_heads, head_dim),
                           &vt);
    if (rc) return rc;
    hipError_t e = ncm::launch_attention_bf16(q, k, v, out, batch, seq_len, q_heads, kv_heads,
                                              head_dim, q_stride, kv_stride, out_stride, window,
                                              out_mode, (uint16_t*)vt, ctx->stream);
    if (e != hipSuccess) return fail_hip(e, "attention launch");
    return NCM_OK;
}

int ncm_attention_bf16_seg_dev(ncm_ctx_t* ctx, const uint16_t* q, const uint16_t* k,
                               const uint16_t* v, void* out, int64_t batch, int64_t seq_len,
                               int q_heads, int kv_heads, int head_dim, int64_t q_stride,
                               int64_t kv_stride, int64_t out_stride, int64_t prefix_len,
                               const int32_t* seg_lo, const int32_t* seg_hi,
                               const uint64_t* prefix_pad_bits, int out_mode) {
    if (!ctx) return NCM_E_NULL;
    if (batch < 0 || seq_len < 0 || q_heads <= 0 || kv_heads <= 0) return NCM_E_SHAPE;
    if (prefix_len < 0 || prefix_len > seq_len) return NCM_E_SHAPE;
    if (head_dim != 64 && head_dim != 128) return NCM_E_SHAPE;
    if (q_heads % kv_heads) return NCM_E_SHAPE;
    if (out_mode != NCM_OUT_BF16_F32 && out_mode != NCM_OUT_BF16) return NCM_E_ARG;
    if (q_stride < (int64_t)q_heads * head_dim || kv_stride < (int64_t)kv_heads * head_dim ||
        out_stride < (int64_t)q_heads * head_dim)
        return NCM_E_SHAPE;
    if (batch == 0 || seq_len == 0) return NCM_OK;
    if (!q || !k || !v || !out || !seg_lo || !seg_hi) return NCM_E_NULL;
    if (q_stride % 8 || kv_stride % 8) return NCM_E_ARG;
    if ((uintptr_t)q % 16 || (uintptr_t)k % 16 || (uintptr_t)v % 16) return NCM_E_ARG;
    if (batch > 65535 || q_heads > 65535 || seq_len > (int64_t(1) << 30)) return NCM_E_SHAPE;
    int rc = ctx_bind(ctx);
    if (rc) return rc;
    void* vt = nullptr;
    rc = ncm_ctx_workspace(ctx, ncm::attention_workspace_bytes(batch, seq_len, kv_heads, head_dim),
                           &vt);
    if (rc) return rc;
    hipError_t e = ncm::launch_attention_bf16_seg(q, k, v, out, batch, seq_len, q_heads, kv_heads,
                                                  head_dim, q_stride, kv_stride, out_stride,
                                                  prefix_len, seg_lo, seg_hi, prefix_pad_bits,
                                                  out_mode, (uint16_t*)vt, ctx->stream);
    if (e != hipSuccess) return fail_hip(e, "attention (level mask) launch");
    return NCM_OK;
}

int ncm_block_diagonal_segments(int64_t prefix_len, const int64_t* level_lengths,
                                int64_t n_levels, const uint8_t* prefix_pad_mask,
                                int64_t pad_len, int64_t seq_len, int32_t* seg_lo,
                                int32_t* seg_hi, uint64_t* pad_bits) {
    if (prefix_len < 0 || n_levels < 0 || seq_len < 0) return NCM_E_SHAPE;
    if (n_levels > 0 && !level_lengths) return NCM_E_NULL;
    // InvalidPrefixMask: a pad mask is empty or one flag per prefix key.
    if (pad_len != 0 && pad_len != prefix_len) return NCM_E_LENGTH;
    if (pad_len > 0 && !prefix_pad_mask) return NCM_E_NULL;
    int64_t total = prefix_len;
    for (int64_t l = 0; l < n_levels; ++l) {
        if (level_lengths[l] < 0 || __builtin_add_overflow(total, level_lengths[l], &total))
            return NCM_E_SHAPE;
    }
    if (total != seq_len) return NCM_E_LENGTH;  // InvalidMaskSize
    if (seq_len > (int64_t(1) << 30)) return NCM_E_SHAPE;
    if (seq_len > 0 && (!seg_lo || !seg_hi)) return NCM_E_NULL;
    for (int64_t t = 0; t < prefix_len; ++t) seg_lo[t] = seg_hi[t] = 0;
    int64_t off = prefix_len;
    for (int64_t l = 0; l < n_levels; ++l) {
        for (int64_t t = off; t < off + level_lengths[l]; ++t) {
            seg_lo[t] = (int32_t)off;
            seg_hi[t] = (int32_t)(off + level_lengths[l]);
        }
        off += level_lengths[l];
    }
    if (pad_bits) {
        for (int64_t w = 0; w < (prefix_len + 63) / 64; ++w) pad_bits[w] = 0;
        for (int64_t t = 0; t < pad_len; ++t)
            if (prefix_pad_mask[t]) pad_bits[t / 64] |= 1ull << (t % 64);
    }
    return NCM_OK;
}

namespace {
// Every layer's required weights present and 16-byte aligned; QK-norm scales
// come in pairs (attention_impl asserts, root.zig:464).
int check_layers(const ncm_decoder_layer_t* layers, int n) {
    for (int l = 0; l < n; ++l) {
        const ncm_decoder_layer_t& L = layers[l];
        if (!L.input_norm || !L.qkv_weight || !L.o_weight || !L.post_attention_norm ||
            !L.gate_up_weight || !L.down_weight)
            return NCM_E_NULL;
        if (!L.q_norm != !L.k_norm) return NCM_E_NULL;
        if ((uintptr_t)L.qkv_weight % 16 || (uintptr_t)L.o_weight % 16 ||
            (uintptr_t)L.gate_up_weight % 16 || (uintptr_t)L.down_weight % 16)
            return NCM_E_ARG;
    }
    return NCM_OK;
}
}  // namespace

int ncm_decoder_forward_dev(ncm_ctx_t* ctx, const ncm_decoder_shape_t* shape,
                            const ncm_decoder_layer_t* layers, const uint16_t* embed,
                            const float* final_norm, const uint16_t* lm_head,
                            const float* cosine, const float* sine, const int64_t* token_ids,
                            int64_t batch, int64_t seq_len, float* logits,
                            const ncm_decoder_trace_t* trace) {
    if (!ctx || !shape) return NCM_E_NULL;
    const ncm_decoder_shape_t& s = *shape;
    if (batch < 0 || seq_len < 0) return NCM_E_SHAPE;
    if (batch == 0 || seq_len == 0) return NCM_E_ARG;  // EmptyInput
    if (s.hidden <= 0 || s.intermediate <= 0 || s.vocab <= 0 || s.layers < 0 || s.window < 0)
        return NCM_E_SHAPE;
    if (s.q_heads <= 0 || s.kv_heads <= 0 || s.q_heads % s.kv_heads) return NCM_E_SHAPE;
    if (s.head_dim != 64 && s.head_dim != 128) return NCM_E_SHAPE;
    if (s.hidden % 8 || s.intermediate % 32) return NCM_E_SHAPE;
    if (s.hidden > (int64_t(1) << 21) || s.intermediate > (int64_t(1) << 20) ||
        s.vocab > (int64_t(1) << 31) || (int64_t)s.q_heads * s.head_dim > (int64_t(1) << 21))
        return NCM_E_SHAPE;
    if (batch > 65535 || batch * seq_len > (int64_t(1) << 31)) return NCM_E_SHAPE;
    if (!embed || !final_norm || !cosine || !sine || !token_ids || !logits) return NCM_E_NULL;
    if (s.layers > 0 && !layers) return NCM_E_NULL;
    if ((uintptr_t)embed % 16 || (lm_head && (uintptr_t)lm_head % 16)) return NCM_E_ARG;
    int rc = check_layers(layers, s.layers);
    if (rc) return rc;
    for (int64_t i = 0; i < batch * seq_len; ++i)
        if (token_ids[i] < 0 || token_ids[i] >= s.vocab) return NCM_E_ARG;  // TokenIdOutOfRange
    rc = ctx_bind(ctx);
    if (rc) return rc;
    void* ws = nullptr;
    rc = ncm_ctx_workspace(ctx, ncm::decoder_workspace_bytes(s, batch, seq_len, trace), &ws);
    if (rc) return rc;
    hipError_t e = ncm::decoder_forward(s, layers, embed, final_norm, lm_head, cosine, sine,
                                        token_ids, batch, seq_len, logits, trace, ws,
                                        ctx->stream);
    if (e != hipSuccess) return fail_hip(e, "decoder forward");
    return NCM_OK;
}

int ncm_decoder_forward_f32_dev(ncm_ctx_t* ctx, const ncm_decoder_shape_t* shape,
                                const ncm_decoder_layer_f32_t* layers, const float* embed,
                                const float* final_norm, const float* lm_head,
                                const float* cosine, const float* sine,
                                const int64_t* token_ids, int64_t batch, int64_t seq_len,
                                float* logits, const ncm_decoder_trace_t* trace) {
    if (!ctx || !shape) return NCM_E_NULL;
    const ncm_decoder_shape_t& s = *shape;
    if (batch < 0 || seq_len < 0) return NCM_E_SHAPE;
    if (batch == 0 || seq_len == 0) return NCM_E_ARG;  // EmptyInput
    if (s.hidden <= 0 || s.intermediate <= 0 || s.vocab <= 0 || s.layers < 0 || s.window < 0)
        return NCM_E_SHAPE;
    if (s.q_heads <= 0 || s.kv_heads <= 0 || s.q_heads % s.kv_heads) return NCM_E_SHAPE;
    // Device limits: 16-byte rows for the fp32 MFMA linear and the attention.
    if (s.head_dim <= 0 || s.head_dim % 4 || s.head_dim > 256) return NCM_E_SHAPE;
    if (s.hidden % 4 || s.intermediate % 4) return NCM_E_SHAPE;
    if (s.hidden > (int64_t(1) << 20) || s.intermediate > (int64_t(1) << 20) ||
        s.vocab > (int64_t(1) << 31) || (int64_t)s.q_heads * s.head_dim > (int64_t(1) << 20))
        return NCM_E_SHAPE;
    if (batch > 65535 || seq_len > (int64_t(1) << 31) - 1 || batch * seq_len > (int64_t(1) << 31))
        return NCM_E_SHAPE;
    if (!embed || !final_norm || !cosine || !sine || !token_ids || !logits) return NCM_E_NULL;
    if (s.layers > 0 && !layers) return NCM_E_NULL;
    if ((uintptr_t)embed % 16 || (lm_head && (uintptr_t)lm_head % 16)) return NCM_E_ARG;
    for (int l = 0; l < s.layers; ++l) {
        const ncm_decoder_layer_f32_t& L = layers[l];
        if (!L.input_norm || !L.qkv_weight || !L.o_weight || !L.post_attention_norm ||
            !L.gate_weight || !L.up_weight || !L.down_weight)
            return NCM_E_NULL;
        if (!L.q_norm != !L.k_norm) return NCM_E_ARG;
        const float* ws_[] = {L.qkv_weight, L.o_weight, L.gate_weight, L.up_weight,
                              L.down_weight};
        for (const float* p : ws_)
            if ((uintptr_t)p % 16) return NCM_E_ARG;
    }
    for (int64_t i = 0; i < batch * seq_len; ++i)
        if (token_ids[i] < 0 || token_ids[i] >= s.vocab) return NCM_E_ARG;  // TokenIdOutOfRange
    int rc = ctx_bind(ctx);
    if (rc) return rc;
    void* ws = nullptr;
    rc = ncm_ctx_workspace(ctx, ncm::decoder_f32_workspace_bytes(s, batch, seq_len), &ws);
    if (rc) return rc;
    hipError_t e = ncm::decoder_forward_f32(s, layers, embed, final_norm, lm_head, cosine, sine,
                                            token_ids, batch, seq_len, logits, trace, ws,
                                            ctx->stream);
    if (e != hipSuccess) return fail_hip(e, "f32 decoder forward");
    return NCM_OK;
}

// The checks of forward_with_trace (src/ncm_model.zig:99-123) in its order,
// then the device path's own limits.
int ncm_ncm_forward_dev(ncm_ctx_t* ctx, const ncm_ncm_shape_t* shape,
                        const ncm_decoder_layer_t* layers, const ncm_ncm_weights_t* weights,
                        const int64_t* prefix_ids, const uint8_t* prefix_pad_mask,
                        int64_t pad_len, const float* target_inputs, const float* cosine,
                        const float* sine, float* output, float* hidden_states) {
    if (!ctx || !shape || !weights) return NCM_E_NULL;
    const ncm_ncm_shape_t& s = *shape;
    if (s.prefix_length < 0 || s.n_levels < 0 || s.n_levels > NCM_MAX_LEVELS) return NCM_E_SHAPE;
    if (pad_len != 0 && pad_len != s.prefix_length) return NCM_E_LENGTH;  // InvalidPrefixMask
    if (s.n_levels == 0) return NCM_E_ARG;                                // InvalidNcmMode
    if (s.hidden <= 0 || s.vq_width <= 0 || s.head_dim <= 0 || s.intermediate <= 0 ||
        s.q_heads <= 0 || s.kv_heads <= 0 || s.head_dim % 2 || s.q_heads % s.kv_heads)
        return NCM_E_SHAPE;  // InvalidNcmDimensions
    if (s.layers <= 0) return NCM_E_LENGTH;  // weights.layers.len == 0: InvalidNcmTensorSize
    if (s.mask_mode < NCM_MASK_BLOCK_DIAGONAL || s.mask_mode > NCM_MASK_CAUSAL || s.window < 0)
        return NCM_E_ARG;
    int64_t S = s.prefix_length;
    for (int l = 0; l < s.n_levels; ++l) {
        if (s.level_lengths[l] < 0 || __builtin_add_overflow(S, s.level_lengths[l], &S))
            return NCM_E_SHAPE;
    }
    // Device limits: the attention kernel's head widths, 16-byte rows.
    if (s.head_dim != 64 && s.head_dim != 128) return NCM_E_SHAPE;
    if (s.hidden % 8 || s.vq_width % 8 || s.intermediate % 32) return NCM_E_SHAPE;
    if (S > (int64_t(1) << 30) || s.hidden > (int64_t(1) << 21) ||
        s.vq_width > (int64_t(1) << 19) || s.intermediate > (int64_t(1) << 20) ||
        (int64_t)s.q_heads * s.head_dim > (int64_t(1) << 21))
        return NCM_E_SHAPE;
    if (S == s.prefix_length) return NCM_E_ARG;  // no target position
    const bool convs = weights->conv_weight || weights->conv_bias;
    if (!weights->prefix_token_embedding && s.prefix_length > 0) return NCM_E_NULL;
    if (!weights->input_projection || !weights->input_projection_bias || !weights->final_norm)
        return NCM_E_NULL;
    if (s.use_level_encoding && !weights->level_embedding) return NCM_E_NULL;
    if (s.query_level0 && !weights->l0_queries && s.level_lengths[0] > 0) return NCM_E_NULL;
    if (convs) {
        if (!weights->conv_weight || !weights->conv_bias) return NCM_E_NULL;
        for (int l = 0; l < s.n_levels; ++l)
            if (!weights->conv_weight[l] || !weights->conv_bias[l]) return NCM_E_NULL;
    }
    if (!target_inputs || !cosine || !sine || !output || !layers) return NCM_E_NULL;
    if (pad_len > 0 && !prefix_pad_mask) return NCM_E_NULL;
    if (s.prefix_length > 0 && !prefix_ids) return NCM_E_NULL;
    if ((uintptr_t)weights->input_projection % 16) return NCM_E_ARG;
    // The convolutions run on the fp32 MFMA's 16-byte loads.
    if (convs)
        for (int l = 0; l < s.n_levels; ++l)
            if ((uintptr_t)weights->conv_weight[l] % 16) return NCM_E_ARG;
    int rc = check_layers(layers, s.layers);
    if (rc) return rc;
    for (int64_t i = 0; i < s.prefix_length; ++i)
        if (prefix_ids[i] < 0 || prefix_ids[i] >= s.prefix_vocab)
            return NCM_E_ARG;  // PrefixTokenOutOfRange
    rc = ctx_bind(ctx);
    if (rc) return rc;
    void* ws = nullptr;
    rc = ncm_ctx_workspace(ctx, ncm::ncm_workspace_bytes(s, convs), &ws);
    if (rc) return rc;
    hipError_t e = ncm::ncm_forward(s, layers, *weights, prefix_ids, prefix_pad_mask, pad_len,
                                    target_inputs, cosine, sine, output, hidden_states, ws,
                                    ctx->stream);
    if (e != hipSuccess) return fail_hip(e, "ncm forward");
    return NCM_OK;
}

// ncm_ncm_forward_f32_dev: the checks of forward_with_trace in its order (as
// ncm_ncm_forward_dev), then the f32 path's device limits.
int ncm_ncm_forward_f32_dev(ncm_ctx_t* ctx, const ncm_ncm_shape_t* shape,
                            const ncm_decoder_layer_f32_t* layers,
                            const ncm_ncm_weights_f32_t* weights, const int64_t* prefix_ids,
                            const uint8_t* prefix_pad_mask, int64_t pad_len,
                            const float* target_inputs, const float* cosine, const float* sine,
                            float* output, float* hidden_states) {
    if (!ctx || !shape || !weights) return NCM_E_NULL;
    const ncm_ncm_shape_t& s = *shape;
    if (s.prefix_length < 0 || s.n_levels < 0 || s.n_levels > NCM_MAX_LEVELS) return NCM_E_SHAPE;
    if (pad_len != 0 && pad_len != s.prefix_length) return NCM_E_LENGTH;  // InvalidPrefixMask
    if (s.n_levels == 0) return NCM_E_ARG;                                // InvalidNcmMode
    if (s.hidden <= 0 || s.vq_width <= 0 || s.head_dim <= 0 || s.intermediate <= 0 ||
        s.q_heads <= 0 || s.kv_heads <= 0 || s.head_dim % 2 || s.q_heads % s.kv_heads)
        return NCM_E_SHAPE;  // InvalidNcmDimensions
    if (s.layers <= 0) return NCM_E_LENGTH;  // InvalidNcmTensorSize
    if (s.mask_mode < NCM_MASK_BLOCK_DIAGONAL || s.mask_mode > NCM_MASK_CAUSAL || s.window < 0)
        return NCM_E_ARG;
    int64_t S = s.prefix_length;
    for (int l = 0; l < s.n_levels; ++l) {
        if (s.level_lengths[l] < 0 || __builtin_add_overflow(S, s.level_lengths[l], &S))
            return NCM_E_SHAPE;
    }
    // Device limits: 16-byte rows for the fp32 MFMA and the attention.
    if (s.head_dim % 4 || s.head_dim > 256) return NCM_E_SHAPE;
    if (s.hidden % 4 || s.vq_width % 4 || s.intermediate % 4) return NCM_E_SHAPE;
    if (S > (int64_t(1) << 30) || s.hidden > (int64_t(1) << 21) ||
        s.vq_width > (int64_t(1) << 19) || s.intermediate > (int64_t(1) << 20) ||
        (int64_t)s.q_heads * s.head_dim > (int64_t(1) << 21))
        return NCM_E_SHAPE;
    if (S == s.prefix_length) return NCM_E_ARG;  // no target position
    const bool convs = weights->conv_weight || weights->conv_bias;
    if (!weights->prefix_token_embedding && s.prefix_length > 0) return NCM_E_NULL;
    if (!weights->input_projection || !weights->final_norm) return NCM_E_NULL;
    if (s.use_level_encoding && !weights->level_embedding) return NCM_E_NULL;
    if (s.query_level0 && !weights->l0_queries && s.level_lengths[0] > 0) return NCM_E_NULL;
    if (convs) {
        if (!weights->conv_weight || !weights->conv_bias) return NCM_E_NULL;
        for (int l = 0; l < s.n_levels; ++l)
            if (!weights->conv_weight[l] || !weights->conv_bias[l]) return NCM_E_NULL;
    }
    if (!target_inputs || !cosine || !sine || !output || !layers) return NCM_E_NULL;
    if (pad_len > 0 && !prefix_pad_mask) return NCM_E_NULL;
    if (s.prefix_length > 0 && !prefix_ids) return NCM_E_NULL;
    if ((uintptr_t)weights->input_projection % 16 || (uintptr_t)target_inputs % 16 ||
        (uintptr_t)output % 16)
        return NCM_E_ARG;
    if (convs)
        for (int l = 0; l < s.n_levels; ++l)
            if ((uintptr_t)weights->conv_weight[l] % 16) return NCM_E_ARG;
    for (int l = 0; l < s.layers; ++l) {
        const ncm_decoder_layer_f32_t& L = layers[l];
        if (!L.input_norm || !L.qkv_weight || !L.o_weight || !L.post_attention_norm ||
            !L.gate_weight || !L.up_weight || !L.down_weight)
            return NCM_E_NULL;
        if (!L.q_norm != !L.k_norm) return NCM_E_ARG;
        const float* ws_[] = {L.qkv_weight, L.o_weight, L.gate_weight, L.up_weight,
                              L.down_weight};
        for (const float* q : ws_)
            if ((uintptr_t)q % 16) return NCM_E_ARG;
    }
    for (int64_t i = 0; i < s.prefix_length; ++i)
        if (prefix_ids[i] < 0 || prefix_ids[i] >= s.prefix_vocab)
            return NCM_E_ARG;  // PrefixTokenOutOfRange
    int rc = ctx_bind(ctx);
    if (rc) return rc;
    void* ws = nullptr;
    rc = ncm_ctx_workspace(ctx, ncm::ncm_f32_workspace_bytes(s, convs), &ws);
    if (rc) return rc;
    hipError_t e = ncm::ncm_forward_f32(s, layers, *weights, prefix_ids, prefix_pad_mask, pad_len,
                                        target_inputs, cosine, sine, output, hidden_states, ws,
                                        ctx->stream);
    if (e != hipSuccess) return fail_hip(e, "ncm forward (f32)");
    return NCM_OK;
}

// ------------------------------------------------------------------ drop-ins

namespace {

// One default context per host thread, created on first use (device 0).
ncm_ctx_t* default_ctx(int* rc) {
    thread_local ncm_ctx_t* ctx = nullptr;
    thread_local int init_rc = 1;
    if (init_rc == 1) init_rc = ncm_init(0, &ctx);
    *rc = init_rc;
    return ctx;
}

size_t align_up(size_t v, size_t a) { return (v + a - 1) / a * a; }

// exact: the reference's own pair-order arithmetic (launch_linear_exact)
// instead of the MFMA linear.
int host_linear(const float* input, size_t input_len, const float* weights, size_t weights_len,
                const float* bias, size_t bias_len, float* output, size_t output_len, size_t T,
                size_t K, size_t N, bool exact = false) {
    // root.zig:107-110: the slice lengths must match the dimensions.
    if (input_len != T * K || weights_len != N * K || output_len != T * N) return NCM_E_LENGTH;
    if (bias && bias_len != N) return NCM_E_LENGTH;
    if (T == 0 || N == 0) return NCM_OK;
    if (!output || (K > 0 && (!input || !weights))) return NCM_E_NULL;
    if (K > (size_t(1) << 21) || T > (size_t(1) << 31) || N > (size_t(1) << 31))
        return NCM_E_SHAPE;
    int rc = 0;
    ncm_ctx_t* ctx = default_ctx(&rc);
    if (rc) return rc;
    rc = ctx_bind(ctx);
    if (rc) return rc;
    // The MFMA path reads rows padded to a multiple of 8 elements; the exact
    // path reads them with stride K.
    const size_t K8 = exact ? K : align_up(K, 8);
    size_t off = 0;
    auto carve = [&](size_t bytes) {
        size_t o = off;
        off = align_up(off + bytes, 256);
        return o;
    };
    const size_t o_xf = carve(T * K * 4), o_wf = carve(N * K * 4), o_bf = carve(N * 4);
    const size_t o_xb = carve(T * K8 * 2), o_wb = carve(N * K8 * 2), o_bb = carve(N * 2);
    const size_t o_y = carve(T * N * 4);
    void* ws = nullptr;
    rc = ncm_ctx_workspace(ctx, off, &ws);
    if (rc) return rc;
    char* base = (char*)ws;
    hipStream_t st = ctx->stream;
    float* xf = (float*)(base + o_xf);
    float* wf = (float*)(base + o_wf);
    float* bf = (float*)(base + o_bf);
    uint16_t* xb = (uint16_t*)(base + o_xb);
    uint16_t* wb = (uint16_t*)(base + o_wb);
    uint16_t* bb = (uint16_t*)(base + o_bb);
    float* y = (float*)(base + o_y);
    if (K > 0) {
        NCM_HIP(hipMemcpyAsync(xf, input, T * K * 4, hipMemcpyHostToDevice, st));
        NCM_HIP(hipMemcpyAsync(wf, weights, N * K * 4, hipMemcpyHostToDevice, st));
    }
    // Operands: round to bf16 and flush subnormals (root.zig:124-135),
    // zero-padding K up to a multiple of 8.
    NCM_HIP(ncm::launch_bf16_from_f32_2d(xf, xb, T, K, K8, 1, st));
    NCM_HIP(ncm::launch_bf16_from_f32_2d(wf, wb, N, K, K8, 1, st));
    if (bias) {
        NCM_HIP(hipMemcpyAsync(bf, bias, N * 4, hipMemcpyHostToDevice, st));
        NCM_HIP(ncm::launch_bf16_from_f32(bf, bb, N, 0, st));  // root.zig:138: no flush
    }
    if (exact)
        NCM_HIP(ncm::launch_linear_exact(xb, wb, bias ? bb : nullptr, y, T, K, N,
                                         NCM_OUT_BF16_F32, st));
    else
        NCM_HIP(ncm::launch_linear(xb, wb, bias ? bb : nullptr, y, T, K8, N, NCM_OUT_BF16_F32, -1,
                                   st));
    NCM_HIP(hipMemcpyAsync(output, y, T * N * 4, hipMemcpyDeviceToHost, st));
    NCM_HIP(hipStreamSynchronize(st));
    return NCM_OK;
}

}  // namespace

int ncm_matmul_f32(const float* input, size_t input_len, const float* weights,
                   size_t weights_len, float* output, size_t output_len, size_t token_count,
                   size_t input_width, size_t output_width) {
    const size_t T = token_count, K = input_width, N = output_width;
    // root.zig:32-34: the slice lengths must match the dimensions.
    if (input_len != T * K || weights_len != N * K || output_len != T * N) return NCM_E_LENGTH;
    if (T == 0 || N == 0) return NCM_OK;
    if (!output || (K > 0 && (!input || !weights))) return NCM_E_NULL;
    if (K > (size_t(1) << 20) || T > (size_t(1) << 31) || N > (size_t(1) << 31))
        return NCM_E_SHAPE;
    int rc = 0;
    ncm_ctx_t* ctx = default_ctx(&rc);
    if (rc) return rc;
    rc = ctx_bind(ctx);
    if (rc) return rc;
    // Rows padded with zeros to K4 = K rounded up to 4 (16-byte rows).
    const size_t K4 = align_up(K, 4);
    const size_t o_x = 0, o_w = align_up(T * K4 * 4, 256), o_y = o_w + align_up(N * K4 * 4, 256);
    void* ws = nullptr;
    rc = ncm_ctx_workspace(ctx, o_y + T * N * 4, &ws);
    if (rc) return rc;
    char* base = (char*)ws;
    hipStream_t st = ctx->stream;
    float* x = (float*)(base + o_x);
    float* w = (float*)(base + o_w);
    float* y = (float*)(base + o_y);
    if (K4 != K) {
        NCM_HIP(hipMemsetAsync(x, 0, T * K4 * 4, st));
        NCM_HIP(hipMemsetAsync(w, 0, N * K4 * 4, st));
    }
    if (K > 0) {
        NCM_HIP(hipMemcpy2DAsync(x, K4 * 4, input, K * 4, K * 4, T, hipMemcpyHostToDevice, st));
        NCM_HIP(hipMemcpy2DAsync(w, K4 * 4, weights, K * 4, K * 4, N, hipMemcpyHostToDevice, st));
    }
    NCM_HIP(ncm::launch_linear_f32(x, w, y, T, K4, N, st));
    NCM_HIP(hipMemcpyAsync(output, y, T * N * 4, hipMemcpyDeviceToHost, st));
    NCM_HIP(hipStreamSynchronize(st));
    return NCM_OK;
}

int ncm_matmul_bf16(const float* input, size_t input_len, const float* weights,
                    size_t weights_len, float* output, size_t output_len, size_t token_count,
                    size_t input_width, size_t output_width) {
    return host_linear(input, input_len, weights, weights_len, nullptr, 0, output, output_len,
                       token_count, input_width, output_width);
}

int ncm_matmul_bf16_bias(const float* input, size_t input_len, const float* weights,
                         size_t weights_len, const float* bias, size_t bias_len, float* output,
                         size_t output_len, size_t token_count, size_t input_width,
                         size_t output_width) {
    if (!bias) return NCM_E_NULL;
    return host_linear(input, input_len, weights, weights_len, bias, bias_len, output,
                       output_len, token_count, input_width, output_width);
}

int ncm_matmul_bf16_exact(const float* input, size_t input_len, const float* weights,
                          size_t weights_len, float* output, size_t output_len,
                          size_t token_count, size_t input_width, size_t output_width) {
    return host_linear(input, input_len, weights, weights_len, nullptr, 0, output, output_len,
                       token_count, input_width, output_width, true);
}

int ncm_matmul_bf16_bias_exact(const float* input, size_t input_len, const float* weights,
                               size_t weights_len, const float* bias, size_t bias_len,
                               float* output, size_t output_len, size_t token_count,
                               size_t input_width, size_t output_width) {
    if (!bias) return NCM_E_NULL;
    return host_linear(input, input_len, weights, weights_len, bias, bias_len, output,
                       output_len, token_count, input_width, output_width, true);
}

int ncm_rms_norm_bf16(const float* input, size_t input_len, const float* weight,
                      size_t weight_len, float* output, size_t output_len, float epsilon) {
    // root.zig:247: nonempty, equal lengths.
    if (input_len == 0 || weight_len != input_len || output_len != input_len)
        return NCM_E_LENGTH;
    if (!input || !weight || !output) return NCM_E_NULL;
    int rc = 0;
    ncm_ctx_t* ctx = default_ctx(&rc);
    if (rc) return rc;
    rc = ctx_bind(ctx);
    if (rc) return rc;
    const size_t n = input_len;
    const size_t o_w = align_up(n * 4, 256), o_y = o_w + align_up(n * 4, 256);
    void* ws = nullptr;
    rc = ncm_ctx_workspace(ctx, o_y + n * 4, &ws);
    if (rc) return rc;
    char* base = (char*)ws;
    hipStream_t st = ctx->stream;
    NCM_HIP(hipMemcpyAsync(base, input, n * 4, hipMemcpyHostToDevice, st));
    NCM_HIP(hipMemcpyAsync(base + o_w, weight, n * 4, hipMemcpyHostToDevice, st));
    NCM_HIP(ncm::launch_rms_norm_rows((const float*)base, (const float*)(base + o_w), base + o_y,
                                      1, (int64_t)n, epsilon, NCM_OUT_BF16_F32, st));
    NCM_HIP(hipMemcpyAsync(output, base + o_y, n * 4, hipMemcpyDeviceToHost, st));
    NCM_HIP(hipStreamSynchronize(st));
    return NCM_OK;
}

int ncm_silu_bf16(const float* input, size_t input_len, float* output, size_t output_len) {
    if (output_len != input_len) return NCM_E_LENGTH;  // root.zig:266
    if (input_len == 0) return NCM_OK;
    if (!input || !output) return NCM_E_NULL;
    int rc = 0;
    ncm_ctx_t* ctx = default_ctx(&rc);
    if (rc) return rc;
    rc = ctx_bind(ctx);
    if (rc) return rc;
    const size_t n = input_len;
    const size_t o_y = align_up(n * 4, 256);
    void* ws = nullptr;
    rc = ncm_ctx_workspace(ctx, o_y + n * 4, &ws);
    if (rc) return rc;
    char* base = (char*)ws;
    hipStream_t st = ctx->stream;
    NCM_HIP(hipMemcpyAsync(base, input, n * 4, hipMemcpyHostToDevice, st));
    NCM_HIP(ncm::launch_silu_mul((const float*)base, nullptr, base + o_y, (int64_t)n,
                                 NCM_OUT_BF16_F32, st));
    NCM_HIP(hipMemcpyAsync(output, base + o_y, n * 4, hipMemcpyDeviceToHost, st));
    NCM_HIP(hipStreamSynchronize(st));
    return NCM_OK;
}

int ncm_round_bf16(const float* values, float* out, size_t n) {
    if (n == 0) return NCM_OK;
    if (!values || !out) return NCM_E_NULL;
    int rc = 0;
    ncm_ctx_t* ctx = default_ctx(&rc);
    if (rc) return rc;
    rc = ctx_bind(ctx);
    if (rc) return rc;
    void* ws = nullptr;
    const size_t o_b = align_up(n * 4, 256);
    rc = ncm_ctx_workspace(ctx, o_b + n * 4 + n * 2 + 256, &ws);
    if (rc) return rc;
    float* f = (float*)ws;
    uint16_t* b = (uint16_t*)((char*)ws + o_b);
    float* w = (float*)((char*)ws + o_b + align_up(n * 2, 256));
    hipStream_t st = ctx->stream;
    NCM_HIP(hipMemcpyAsync(f, values, n * 4, hipMemcpyHostToDevice, st));
    NCM_HIP(ncm::launch_bf16_from_f32(f, b, (int64_t)n, 0, st));
    NCM_HIP(ncm::launch_bf16_widen(b, w, (int64_t)n, st));
    NCM_HIP(hipMemcpyAsync(out, w, n * 4, hipMemcpyDeviceToHost, st));
    NCM_HIP(hipStreamSynchronize(st));
    return NCM_OK;
}

// ------------------------------------------------------------------ RVQ

int ncm_rvq_prepare(ncm_ctx_t* ctx, const uint16_t* codebooks, int64_t levels, int64_t v,
                    int64_t d, float* csq) {
    if (!ctx) return NCM_E_NULL;
    if (levels < 1 || v < 1 || d < 1) return NCM_E_SHAPE;
    if (!codebooks || !csq) return NCM_E_NULL;
    int rc = ctx_bind(ctx);
    if (rc) return rc;
    hipError_t e = ncm::launch_rvq_csq(codebooks, levels * v, d, csq, ctx->stream);
    if (e != hipSuccess) return fail_hip(e, "rvq csq launch");
    return NCM_OK;
}

int ncm_rvq_encode(ncm_ctx_t* ctx, const float* x, int64_t b, int64_t t, int64_t d,
                   int64_t levels, const int32_t* strides, const uint16_t* codebooks,
                   const float* csq, int64_t v, int32_t* codes, float* recon, float* gap,
                   const int32_t* force_codes, int64_t* n_flagged) {
    if (!ctx) return NCM_E_NULL;
    if (!x || !strides || !codebooks || !csq || !codes) return NCM_E_NULL;
    int rc = ncm::rvq_check_shape(b, t, d, levels, strides, v);
    if (rc) return rc;
    rc = ctx_bind(ctx);
    if (rc) return rc;
    return ncm::rvq_encode(ctx, x, b, t, d, levels, strides, codebooks, csq, v, codes, recon,
                           gap, force_codes, n_flagged);
}

int ncm_rvq_encode_counts(ncm_ctx_t* ctx, const float* x, int64_t b, int64_t t, int64_t d,
                          int64_t levels, const int32_t* strides, const uint16_t* codebooks,
                          const float* csq, int64_t v, int32_t* codes, float* recon, float* gap,
                          const int32_t* force_codes, int64_t* flagged, int64_t* scored) {
    if (!ctx) return NCM_E_NULL;
    if (!x || !strides || !codebooks || !csq || !codes || !flagged || !scored) return NCM_E_NULL;
    int rc = ncm::rvq_check_shape(b, t, d, levels, strides, v);
    if (rc) return rc;
    rc = ctx_bind(ctx);
    if (rc) return rc;
    ncm::RvqCounts counts{};
    rc = ncm::rvq_encode(ctx, x, b, t, d, levels, strides, codebooks, csq, v, codes, recon, gap,
                         force_codes, nullptr, &counts);
    if (rc) return rc;
    for (int64_t l = 0; l < levels; ++l) {
        flagged[l] = counts.flagged[l];
        scored[l] = counts.scored[l];
    }
    return NCM_OK;
}

// Shape, switch and weight checks shared by the tokenizer entry points.
static int vq_tok_check(const ncm_vq_tok_t* t, bool need_embed) {
    if (!t) return NCM_E_NULL;
    if (t->n_levels < 1 || t->n_levels > NCM_VQ_TOK_MAX_LEVELS) return NCM_E_SHAPE;
    if (t->groups < 1 || t->embed_dim <= 0 || t->embed_dim % (4 * t->groups) ||
        t->embed_dim > (1 << 16))
        return NCM_E_SHAPE;
    const int64_t L = t->level_len[t->n_levels - 1];
    if (L < 1 || L > (1 << 20)) return NCM_E_SHAPE;
    for (int l = 0; l < t->n_levels; ++l) {
        if (t->level_len[l] < 1 || t->level_len[l] > L) return NCM_E_SHAPE;
        if (l > 0 && t->level_len[l] <= t->level_len[l - 1]) return NCM_E_SHAPE;
        if (t->level_vocab[l] < 1 || t->level_vocab[l] > (int64_t(1) << 30)) return NCM_E_SHAPE;
        if (!t->codebook[l]) return NCM_E_NULL;
        if ((uintptr_t)t->codebook[l] % 16) return NCM_E_ARG;
        if (t->resi_weight[l] && (!t->resi_bias[l] || (uintptr_t)t->resi_weight[l] % 16))
            return NCM_E_ARG;
    }
    if (t->learned_level0) {
        if (t->n_stages < 0 || t->n_stages > NCM_VQ_TOK_MAX_STAGES) return NCM_E_SHAPE;
        if (L % t->level_len[0]) return NCM_E_SHAPE;
        int64_t prod = 1;
        for (int i = 0; i < t->n_stages; ++i) {
            if (t->stage_stride[i] < 1 || t->stage_stride[i] > 64) return NCM_E_SHAPE;
            prod *= t->stage_stride[i];
            if (!t->down_weight[i] || !t->down_bias[i] || !t->up_weight[i] || !t->up_bias[i])
                return NCM_E_NULL;
            if ((uintptr_t)t->down_weight[i] % 16 || (uintptr_t)t->up_weight[i] % 16)
                return NCM_E_ARG;
        }
        if (prod != L / t->level_len[0]) return NCM_E_SHAPE;
    }
    if (need_embed) {
        if (!t->wte || !t->wpe) return NCM_E_NULL;
        if ((uintptr_t)t->wte % 16 || (uintptr_t)t->wpe % 16) return NCM_E_ARG;
        if (t->in_vocab < 1 || t->in_vocab > (int64_t(1) << 31) || t->context_length < L)
            return NCM_E_SHAPE;
        if (!(t->group_eps >= 0.0f)) return NCM_E_ARG;
    }
    return NCM_OK;
}

static int vq_tok_batch_ok(const ncm_vq_tok_t* t, int64_t batch) {
    if (batch < 0) return NCM_E_SHAPE;
    if (batch == 0) return NCM_E_ARG;  // EmptyInput
    if (batch > 65535) return NCM_E_SHAPE;
    int64_t nsum = 0;
    for (int l = 0; l < t->n_levels; ++l) nsum += t->level_len[l];
    const int64_t L = t->level_len[t->n_levels - 1];
    // Activation buffers below 2^31 elements, codes below 2^31 entries.
    if (batch * (L + 2) * t->embed_dim >= (int64_t(1) << 31) || batch * nsum >= (int64_t(1) << 31))
        return NCM_E_SHAPE;
    return NCM_OK;
}

static int vq_tok_run(ncm_ctx_t* ctx, const ncm_vq_tok_t* tok, const int32_t* ids,
                      const float* latent_in, int64_t batch, int32_t* codes, float* zhat,
                      float* latent_out) {
    int rc = ctx_bind(ctx);
    if (rc) return rc;
    void* ws = nullptr;
    rc = ncm_ctx_workspace(ctx, ncm::vq_tok_workspace_bytes(*tok, batch, zhat == nullptr), &ws);
    if (rc) return rc;
    hipError_t e = ncm::vq_tok_encode(*tok, ids, latent_in, batch, codes, zhat, latent_out, ws,
                                      ctx->stream);
    if (e != hipSuccess) return fail_hip(e, "vq tokenizer encode");
    return NCM_OK;
}

int ncm_vq_tok_pack_conv_dev(ncm_ctx_t* ctx, const float* src, float* dst, int64_t c, int64_t k,
                             int transposed) {
    if (!ctx) return NCM_E_NULL;
    if (!src || !dst) return NCM_E_NULL;
    if (c <= 0 || k <= 0 || c > (1 << 16) || k > 64) return NCM_E_SHAPE;
    if (transposed != 0 && transposed != 1) return NCM_E_ARG;
    int rc = ctx_bind(ctx);
    if (rc) return rc;
    hipError_t e = ncm::vq_tok_pack_conv(src, dst, c, k, transposed, ctx->stream);
    if (e != hipSuccess) return fail_hip(e, "vq tokenizer conv pack");
    return NCM_OK;
}

int ncm_vq_tok_encode_dev(ncm_ctx_t* ctx, const ncm_vq_tok_t* tok, const int64_t* token_ids,
                          int64_t batch, int32_t* codes, float* zhat, float* latent) {
    if (!ctx) return NCM_E_NULL;
    int rc = vq_tok_check(tok, true);
    if (rc) return rc;
    rc = vq_tok_batch_ok(tok, batch);
    if (rc) return rc;
    if (!token_ids || !codes) return NCM_E_NULL;
    if ((zhat && (uintptr_t)zhat % 16) || (latent && (uintptr_t)latent % 16)) return NCM_E_ARG;
    const int64_t L = tok->level_len[tok->n_levels - 1];
    std::vector<int32_t> ids((size_t)(batch * L));
    for (int64_t i = 0; i < batch * L; ++i) {
        if (token_ids[i] < 0 || token_ids[i] >= tok->in_vocab) return NCM_E_ARG;
        ids[(size_t)i] = (int32_t)token_ids[i];
    }
    return vq_tok_run(ctx, tok, ids.data(), nullptr, batch, codes, zhat, latent);
}

int ncm_vq_tok_quantize_dev(ncm_ctx_t* ctx, const ncm_vq_tok_t* tok, const float* latent,
                            int64_t batch, int32_t* codes, float* zhat) {
    if (!ctx) return NCM_E_NULL;
    int rc = vq_tok_check(tok, false);
    if (rc) return rc;
    rc = vq_tok_batch_ok(tok, batch);
    if (rc) return rc;
    if (!latent || !codes) return NCM_E_NULL;
    if ((uintptr_t)latent % 16 || (zhat && (uintptr_t)zhat % 16)) return NCM_E_ARG;
    return vq_tok_run(ctx, tok, nullptr, latent, batch, codes, zhat, nullptr);
}

int ncm_vq_tok_reconstruct_dev(ncm_ctx_t* ctx, const ncm_vq_tok_t* tok, const int32_t* codes,
                               int64_t batch, float* zhat) {
    if (!ctx) return NCM_E_NULL;
    int rc = vq_tok_check(tok, false);
    if (rc) return rc;
    rc = vq_tok_batch_ok(tok, batch);
    if (rc) return rc;
    if (!codes || !zhat) return NCM_E_NULL;
    if ((uintptr_t)zhat % 16) return NCM_E_ARG;
    rc = ctx_bind(ctx);
    if (rc) return rc;
    void* ws = nullptr;
    rc = ncm_ctx_workspace(ctx, ncm::vq_tok_workspace_bytes(*tok, batch, false), &ws);
    if (rc) return rc;
    hipError_t e = ncm::vq_tok_reconstruct(*tok, codes, batch, zhat, ws, ctx->stream);
    if (e != hipSuccess) return fail_hip(e, "vq tokenizer reconstruct");
    return NCM_OK;
}

int ncm_vq_tok_decode_dev(ncm_ctx_t* ctx, const ncm_vq_tok_t* tok,
                          const ncm_vq_tok_decoder_t* dec, const float* zhat, int64_t batch,
                          float* logits) {
    if (!ctx || !tok || !dec) return NCM_E_NULL;
    if (tok->n_levels < 1 || tok->n_levels > NCM_VQ_TOK_MAX_LEVELS) return NCM_E_SHAPE;
    const int64_t L = tok->level_len[tok->n_levels - 1], D = tok->embed_dim;
    const int64_t C = tok->in_vocab;
    if (L < 1 || L > 4096 || D < 4 || D % 4 || D > (1 << 16) || C < 1 || C % 4 ||
        C > (int64_t(1) << 31))
        return NCM_E_SHAPE;
    if (dec->n_head < 1 || D % dec->n_head || (D / dec->n_head) % 4 || D / dec->n_head > 256)
        return NCM_E_SHAPE;
    if (batch < 0) return NCM_E_SHAPE;
    if (batch == 0) return NCM_E_ARG;
    if (batch > 65535 || batch * L * 4 * D >= (int64_t(1) << 31) ||
        batch * L * C >= (int64_t(1) << 40))
        return NCM_E_SHAPE;
    if (!zhat || !logits) return NCM_E_NULL;
    if (!dec->ln1_weight || !dec->attn_weight || !dec->proj_weight || !dec->ln2_weight ||
        !dec->fc_weight || !dec->fc_proj_weight || !dec->lnf_weight || !dec->out_weight)
        return NCM_E_NULL;
    if (!dec->q_norm != !dec->k_norm) return NCM_E_ARG;
    if (!(dec->ln_eps >= 0.0f) || !(dec->qk_eps >= 0.0f)) return NCM_E_ARG;
    const void* al[] = {zhat, logits, dec->ln1_weight, dec->ln1_bias, dec->attn_weight,
                        dec->proj_weight, dec->ln2_weight, dec->ln2_bias, dec->fc_weight,
                        dec->fc_proj_weight, dec->lnf_weight, dec->out_weight};
    for (const void* q : al)
        if ((uintptr_t)q % 16) return NCM_E_ARG;
    int rc = ctx_bind(ctx);
    if (rc) return rc;
    void* ws = nullptr;
    rc = ncm_ctx_workspace(ctx, ncm::vq_tok_decoder_workspace_bytes(*tok, batch), &ws);
    if (rc) return rc;
    hipError_t e = ncm::vq_tok_decode(*tok, *dec, zhat, batch, logits, ws, ctx->stream);
    if (e != hipSuccess) return fail_hip(e, "vq tokenizer decode");
    return NCM_OK;
}

int ncm_rvq_decode(ncm_ctx_t* ctx, const int32_t* codes, int64_t b, int64_t t, int64_t d,
                   int64_t levels, const int32_t* strides, const uint16_t* codebooks, int64_t v,
                   float* recon) {
    if (!ctx) return NCM_E_NULL;
    if (!codes || !strides || !codebooks || !recon) return NCM_E_NULL;
    int rc = ncm::rvq_check_shape(b, t, d, levels, strides, v);
    if (rc) return rc;
    rc = ctx_bind(ctx);
    if (rc) return rc;
    hipError_t e = ncm::launch_rvq_decode(codes, b, t, d, levels, strides, codebooks, v, recon,
                                          ctx->stream);
    if (e != hipSuccess) return fail_hip(e, "rvq decode launch");
    return NCM_OK;
}

}  // extern "C"
