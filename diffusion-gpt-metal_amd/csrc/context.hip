// Context lifecycle and dispatch-region semantics of the C ABI
// (mirrors src/GPU.swift:118-198: init, begin, end, go's bookkeeping).
#include <cstdarg>
#include <mutex>
#include <new>

#include "common.hpp"

namespace {

// Scratch of the allocation-free entry point (dgm_gemmNT_noalloc): every
// device holds its own copy from library load to process end. Host code uses
// only the per-device address from hipGetSymbolAddress, never this name.
__device__ __align__(256) uint8_t scratch[dgm::kScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex scratch_mu;
void* scratch_addr[kMaxDevices] = {};

// The device address of `scratch` on `device` (current), resolved once per
// device. Returns nullptr (and the HIP error) when it cannot be resolved.
void* scratch_for(int device, hipError_t* err) {
    *err = hipSuccess;
    if (device < 0 || device >= kMaxDevices) {
        *err = hipErrorInvalidDevice;
        return nullptr;
    }
    std::lock_guard<std::mutex> lock(scratch_mu);
    if (!scratch_addr[device]) {
        void* p = nullptr;
        *err = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (*err != hipSuccess) return nullptr;
        scratch_addr[device] = p;
    }
    return scratch_addr[device];
}

}  // namespace

namespace dgm {

int fail(dgm_gpu* g, int code, const char* fmt, ...) {
    if (!g) return code;
    if (g->first_err == DGM_OK) {
        g->first_err = code;
        va_list ap;
        va_start(ap, fmt);
        vsnprintf(g->err_msg, sizeof(g->err_msg), fmt, ap);
        va_end(ap);
    }
    return code;
}

int enter(dgm_gpu* g, const char* name) {
    if (!g) return DGM_ERR_ARG;
    // GPU.go (src/GPU.swift:183): dispatching outside begin()/end() is a
    // programming error in the reference (fatalError); here it is a status.
    if (!g->begun) return fail(g, DGM_ERR_NOT_BEGUN, "begin() was not called before %s", name);
    snprintf(g->last_kernel, sizeof(g->last_kernel), "%s", name);
    return DGM_OK;
}

int check_launch(dgm_gpu* g, const char* name) {
    hipError_t e = hipGetLastError();
    if (e != hipSuccess)
        return fail(g, DGM_ERR_HIP, "launch of %s failed: %s", name, hipGetErrorString(e));
    return DGM_OK;
}

void* workspace(dgm_gpu* g, size_t bytes) {
    if (g->use_scratch) {
        // dgm_gemmNT_noalloc: the static scratch or nothing, never hipMalloc.
        if (!g->scratch) {
            fail(g, DGM_ERR_HIP, "the static scratch of device %d could not be resolved", g->device);
            return nullptr;
        }
        if (bytes > kScratchBytes) {
            fail(g, DGM_ERR_UNSUPPORTED, "this call needs %zu bytes of scratch; the static scratch holds %zu", bytes,
                 kScratchBytes);
            return nullptr;
        }
        return g->scratch;
    }
    if (bytes <= g->ws_bytes) return g->ws;
    // Growing inside a graph capture would bake a fresh allocation into the
    // graph (and hipMalloc is not capturable): refuse, and let the caller make
    // one such call before capturing.
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(g->stream, &cs) == hipSuccess && cs != hipStreamCaptureStatusNone) {
        fail(g, DGM_ERR_UNSUPPORTED,
             "workspace would grow to %zu bytes during graph capture; run one such call before capturing", bytes);
        return nullptr;
    }
    if (g->n_retired == dgm_gpu::kMaxRetired) {
        fail(g, DGM_ERR_UNSUPPORTED, "workspace grew %d times; the context keeps every retired buffer",
             dgm_gpu::kMaxRetired);
        return nullptr;
    }
    // At least double, so the retired buffers total less than the live one.
    size_t want = bytes < 2 * g->ws_bytes ? 2 * g->ws_bytes : bytes;
    if (want < (size_t(1) << 20)) want = size_t(1) << 20;
    void* p = nullptr;
    if (hipMalloc(&p, want) != hipSuccess) {
        fail(g, DGM_ERR_HIP, "workspace allocation of %zu bytes failed", want);
        return nullptr;
    }
    // The old buffer is not freed here: work still queued on any stream and
    // graphs captured earlier may read or write it. It lives until
    // dgm_gpu_destroy.
    if (g->ws) g->retired[g->n_retired++] = g->ws;
    g->ws = p;
    g->ws_bytes = want;
    return g->ws;
}

int ws_error(dgm_gpu* g) { return g->first_err != DGM_OK ? g->first_err : DGM_ERR_HIP; }

}  // namespace dgm

extern "C" {

int dgm_gpu_create(dgm_gpu** out) {
    if (!out) return DGM_ERR_ARG;
    *out = nullptr;
    dgm_gpu* g = new (std::nothrow) dgm_gpu();
    if (!g) return DGM_ERR_ARG;
    if (hipGetDevice(&g->device) != hipSuccess) { delete g; return DGM_ERR_HIP; }
    hipDeviceProp_t prop;
    if (hipGetDeviceProperties(&prop, g->device) == hipSuccess && prop.multiProcessorCount > 0)
        g->num_cus = prop.multiProcessorCount;
    // The allocation-free entry point's scratch on this device (resolved once
    // per device; a failure surfaces only when that entry point is called).
    hipError_t se;
    g->scratch = scratch_for(g->device, &se);
    // A blocking stream: it orders itself after work on the null stream, where
    // callers that allocate with torch or hipMemset may still be filling the
    // buffers they hand over.
    if (hipStreamCreateWithFlags(&g->own_stream, hipStreamDefault) != hipSuccess) {
        delete g;
        return DGM_ERR_HIP;
    }
    g->stream = g->own_stream;
    *out = g;
    return DGM_OK;
}

void dgm_gpu_destroy(dgm_gpu* g) {
    if (!g) return;
    // Work queued by this context may still use its workspace: wait for the
    // streams it launched on (not the whole device, where another thread may
    // be capturing a graph).
    if (g->stream) (void)hipStreamSynchronize(g->stream);
    if (g->own_stream && g->own_stream != g->stream) (void)hipStreamSynchronize(g->own_stream);
    for (int i = 0; i < g->n_streams; ++i)
        if (g->streams[i] != g->stream) (void)hipStreamSynchronize(g->streams[i]);
    if (g->many_streams) (void)hipDeviceSynchronize();
    if (g->ws) (void)hipFree(g->ws);
    for (int i = 0; i < g->n_retired; ++i) (void)hipFree(g->retired[i]);
    if (g->own_stream) (void)hipStreamDestroy(g->own_stream);
    delete g;
}

int dgm_gpu_set_stream(dgm_gpu* g, void* hip_stream) {
    if (!g) return DGM_ERR_ARG;
    hipStream_t s = hip_stream ? static_cast<hipStream_t>(hip_stream) : g->own_stream;
    if (s != g->own_stream) {
        bool known = false;
        for (int i = 0; i < g->n_streams; ++i) known = known || g->streams[i] == s;
        if (!known) {
            if (g->n_streams < dgm_gpu::kMaxStreams) g->streams[g->n_streams++] = s;
            else g->many_streams = true;   // destroy then waits for the whole device
        }
    }
    g->stream = s;
    return DGM_OK;
}

void* dgm_gpu_stream(const dgm_gpu* g) { return g ? static_cast<void*>(g->stream) : nullptr; }

int dgm_set_math(dgm_gpu* g, int mode) {
    if (!g) return DGM_ERR_ARG;
    if (mode != DGM_MATH_FP32 && mode != DGM_MATH_BF16) return DGM_ERR_ARG;
    g->math = mode;
    return DGM_OK;
}

int dgm_get_math(const dgm_gpu* g) { return g ? g->math : -1; }

int dgm_begin(dgm_gpu* g) {
    if (!g) return DGM_ERR_ARG;
    g->begun = true;
    g->first_err = DGM_OK;
    g->err_msg[0] = 0;
    return DGM_OK;
}

int dgm_end(dgm_gpu* g) {
    if (!g) return DGM_ERR_ARG;
    g->begun = false;
    hipError_t e = hipStreamSynchronize(g->stream);
    if (e == hipSuccess) e = hipGetLastError();
    if (e != hipSuccess)
        dgm::fail(g, DGM_ERR_HIP, "HIP error after %s: %s", g->last_kernel, hipGetErrorString(e));
    else if (g->spin_waits)
        dgm::decode_wait_check(g);
    return g->first_err;
}

const char* dgm_last_kernel(const dgm_gpu* g) { return g ? g->last_kernel : ""; }
const char* dgm_last_error(const dgm_gpu* g) { return g ? g->err_msg : ""; }

}  // extern "C"
