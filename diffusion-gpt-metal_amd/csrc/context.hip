// Context lifecycle and dispatch-region semantics of the C ABI
// (mirrors src/GPU.swift:118-198: init, begin, end, go's bookkeeping).
#include <cstdarg>
#include <new>

#include "common.hpp"

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
    if (bytes <= g->ws_bytes) return g->ws;
    // Work already queued may still read the old buffer.
    if (g->ws) {
        (void)hipStreamSynchronize(g->stream);
        (void)hipFree(g->ws);
        g->ws = nullptr;
        g->ws_bytes = 0;
    }
    size_t want = bytes < (size_t(1) << 20) ? (size_t(1) << 20) : bytes;
    if (hipMalloc(&g->ws, want) != hipSuccess) {
        g->ws = nullptr;
        fail(g, DGM_ERR_HIP, "workspace allocation of %zu bytes failed", want);
        return nullptr;
    }
    g->ws_bytes = want;
    return g->ws;
}

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
    if (g->stream) (void)hipStreamSynchronize(g->stream);
    if (g->ws) (void)hipFree(g->ws);
    if (g->own_stream) (void)hipStreamDestroy(g->own_stream);
    delete g;
}

int dgm_gpu_set_stream(dgm_gpu* g, void* hip_stream) {
    if (!g) return DGM_ERR_ARG;
    g->stream = hip_stream ? static_cast<hipStream_t>(hip_stream) : g->own_stream;
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
    return g->first_err;
}

const char* dgm_last_kernel(const dgm_gpu* g) { return g ? g->last_kernel : ""; }
const char* dgm_last_error(const dgm_gpu* g) { return g ? g->err_msg : ""; }

}  // extern "C"
