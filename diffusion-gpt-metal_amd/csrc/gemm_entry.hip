// C-ABI entry points of the GEMM family and the GPU.swift-style wrappers
// (src/GPU.swift:227-272). Validates the reference's preconditions, then hands
// the call to the router of its direction (gemm_f32.hip): for quantized
// forwards the few-row and decode-shaped kernels (int8 / f16 / bf16 MFMA over
// exact activation pieces), the bf16 prefill kernel in the reduced-precision
// mode, else the fp32 MFMA tiles; dX and dW always on the fp32 tiles.
#include "common.hpp"

#include <algorithm>

namespace dgm {
int gemm_check_sizes(dgm_gpu* g, const char* name, const dgm_GemmP* p, int bits);
int gemm_f32_fwd(dgm_gpu* g, int bits, const void* W, const float* scale, const float* X,
                 const float* bias, float* Y, const dgm_GemmP* p);
int gemm_f32_dx(dgm_gpu* g, int bits, const void* W, const float* scale, const float* dY,
                float* dX, const dgm_GemmP* p);
int gemm_f32_dw(dgm_gpu* g, const float* dY, const float* X, float* dW, const dgm_GemmP* p,
                bool accumulate);
int gemm_f32_bwd_pair(dgm_gpu* g, int bits, const void* W, const float* scale, const float* dY, const float* X,
                      float* dX, float* dW, const dgm_GemmP* p, bool accumulate, bool* fused,
                      const float* sg_gate = nullptr, const float* sg_up = nullptr);
}  // namespace dgm

namespace {

int gemm_nt(dgm_gpu* g, const char* name, int bits, const void* W, const float* scale,
            const float* X, const float* bias, float* Y, const dgm_GemmP* p) {
    int rc = dgm::enter(g, name);
    if (rc) return rc;
    rc = dgm::gemm_check_sizes(g, name, p, bits);
    if (rc) return rc;
    if (p->M == 0 || p->N == 0) return DGM_OK;
    if (!Y || (p->K > 0 && (!W || !X)) || (bits != 32 && p->K > 0 && !scale) ||
        (p->hasBias && !bias))
        return dgm::fail(g, DGM_ERR_ARG, "%s: null buffer", name);
    rc = dgm::gemm_f32_fwd(g, bits, W, scale, X, bias, Y, p);
    if (rc) return rc;
    DGM_LAUNCH_CHECK(g, name);
    return DGM_OK;
}

int gemm_dx(dgm_gpu* g, const char* name, int bits, const void* W, const float* scale,
            const float* dY, float* dX, const dgm_GemmP* p) {
    int rc = dgm::enter(g, name);
    if (rc) return rc;
    rc = dgm::gemm_check_sizes(g, name, p, bits);
    if (rc) return rc;
    if (p->M == 0 || p->K == 0) return DGM_OK;
    if (!dX || (p->N > 0 && (!W || !dY)) || (bits != 32 && p->N > 0 && !scale))
        return dgm::fail(g, DGM_ERR_ARG, "%s: null buffer", name);
    rc = dgm::gemm_f32_dx(g, bits, W, scale, dY, dX, p);
    if (rc) return rc;
    DGM_LAUNCH_CHECK(g, name);
    return DGM_OK;
}

int gemm_dw(dgm_gpu* g, const char* name, const float* dY, const float* X, float* dW,
            const dgm_GemmP* p, bool accumulate) {
    int rc = dgm::enter(g, name);
    if (rc) return rc;
    rc = dgm::gemm_check_sizes(g, name, p, 32);
    if (rc) return rc;
    if (p->N == 0 || p->K == 0) return DGM_OK;
    if (!dW || (p->M > 0 && (!dY || !X))) return dgm::fail(g, DGM_ERR_ARG, "%s: null buffer", name);
    rc = dgm::gemm_f32_dw(g, dY, X, dW, p, accumulate);
    if (rc) return rc;
    DGM_LAUNCH_CHECK(g, name);
    return DGM_OK;
}

int make_p(dgm_gpu* g, const char* name, int64_t M, int64_t N, int64_t K, int hasBias,
           int64_t qGroup, dgm_GemmP* p) {
    if (M < 0 || N < 0 || K < 0 || M > dgm::kMaxIndex || N > dgm::kMaxIndex || K > dgm::kMaxIndex ||
        qGroup < 0 || qGroup > dgm::kMaxIndex)
        return dgm::fail(g, DGM_ERR_ARG, "%s: bad sizes M=%lld N=%lld K=%lld group=%lld", name,
                         (long long)M, (long long)N, (long long)K, (long long)qGroup);
    *p = dgm_GemmP{uint32_t(M), uint32_t(N), uint32_t(K), uint32_t(hasBias), uint32_t(qGroup), 0, 0, 0};
    return DGM_OK;
}

}  // namespace

extern "C" {

int dgm_gemm_nt_f32(dgm_gpu* g, const float* W, const float* X, const float* bias, float* Y,
                    const dgm_GemmP* p) {
    return gemm_nt(g, "gemm_nt_f32", 32, W, nullptr, X, bias, Y, p);
}
int dgm_gemm_nt_i8(dgm_gpu* g, const int8_t* W, const float* scale, const float* X,
                   const float* bias, float* Y, const dgm_GemmP* p) {
    return gemm_nt(g, "gemm_nt_i8", 8, W, scale, X, bias, Y, p);
}
int dgm_gemm_nt_i4(dgm_gpu* g, const uint8_t* W, const float* scale, const float* X,
                   const float* bias, float* Y, const dgm_GemmP* p) {
    return gemm_nt(g, "gemm_nt_i4", 4, W, scale, X, bias, Y, p);
}
int dgm_gemm_dx_f32(dgm_gpu* g, const float* W, const float* dY, float* dX, const dgm_GemmP* p) {
    return gemm_dx(g, "gemm_dx_f32", 32, W, nullptr, dY, dX, p);
}
int dgm_gemm_dx_i8(dgm_gpu* g, const int8_t* W, const float* scale, const float* dY, float* dX,
                   const dgm_GemmP* p) {
    return gemm_dx(g, "gemm_dx_i8", 8, W, scale, dY, dX, p);
}
int dgm_gemm_dx_i4(dgm_gpu* g, const uint8_t* W, const float* scale, const float* dY, float* dX,
                   const dgm_GemmP* p) {
    return gemm_dx(g, "gemm_dx_i4", 4, W, scale, dY, dX, p);
}
int dgm_gemm_dw(dgm_gpu* g, const float* dY, const float* X, float* dW, const dgm_GemmP* p) {
    return gemm_dw(g, "gemm_dw", dY, X, dW, p, false);
}
int dgm_gemm_dw_acc(dgm_gpu* g, const float* dY, const float* X, float* dW, const dgm_GemmP* p) {
    return gemm_dw(g, "gemm_dw_acc", dY, X, dW, p, true);
}

int dgm_gemmNT(dgm_gpu* g, int64_t bits, const float* w, const void* q, const float* scale,
               const float* x, const float* bias, float* y, int64_t M, int64_t N, int64_t K,
               int64_t qGroup) {
    if (!g) return DGM_ERR_ARG;
    dgm_GemmP p;
    int rc = make_p(g, "gemmNT", M, N, K, bias ? 1 : 0, qGroup, &p);
    if (rc) return rc;
    switch (bits) {
        case 32: return dgm_gemm_nt_f32(g, w, x, bias, y, &p);
        case 8: return dgm_gemm_nt_i8(g, static_cast<const int8_t*>(q), scale, x, bias, y, &p);
        case 4: return dgm_gemm_nt_i4(g, static_cast<const uint8_t*>(q), scale, x, bias, y, &p);
        default: return dgm::fail(g, DGM_ERR_BITS, "gemmNT: unsupported bits %lld", (long long)bits);
    }
}

int dgm_gemmNT_noalloc(dgm_gpu* g, int64_t bits, const float* w, const void* q, const float* scale,
                       const float* x, const float* bias, float* y, int64_t M, int64_t N, int64_t K, int64_t qGroup) {
    // dgm_gemmNT with every staging buffer taken from the static device
    // scratch: nothing is allocated, and a call that would need more than
    // kScratchBytes fails with DGM_ERR_UNSUPPORTED before launching anything.
    if (!g) return DGM_ERR_ARG;
    g->use_scratch = true;
    const int rc = dgm_gemmNT(g, bits, w, q, scale, x, bias, y, M, N, K, qGroup);
    g->use_scratch = false;
    return rc;
}

int64_t dgm_gemmNT_workspace_bound(int64_t M, int64_t N, int64_t K) {
    if (M < 0 || N < 0 || K < 0) return -1;
    // Activation pieces of the decode-shaped kernels (M <= 64 and the int8
    // skinny kernel's virtual rows): at most 4 row tiles x 2 pieces x 1 KB per
    // 32 k, plus the exponents / offset terms (4 bytes per row tile, 16 rows,
    // per 64 k) and alignment slack.
    int64_t b = 260 * K + 512;
    // bf16 copy of X (reduced-precision prefill, M > 64).
    if (M > 64) b = std::max(b, 2 * M * K);
    // Partial sums of the K-sliced kernel (M <= 16): slices x M x N floats with
    // at most K / 256 slices, refused beyond the static scratch's size.
    if (M <= 16) b = std::max(b, std::min<int64_t>(int64_t(dgm::kScratchBytes), M * N * (K / 256) * 4));
    return b;
}

int dgm_gpu_reserve(dgm_gpu* g, int64_t bytes) {
    if (!g || bytes < 0) return DGM_ERR_ARG;
    if (size_t(bytes) <= g->ws_bytes) return DGM_OK;
    return dgm::workspace(g, size_t(bytes)) ? DGM_OK : dgm::ws_error(g);
}

int64_t dgm_gpu_workspace_bytes(const dgm_gpu* g) { return g ? int64_t(g->ws_bytes) : -1; }

int dgm_gemmDX(dgm_gpu* g, int64_t bits, const float* w, const void* q, const float* scale,
               const float* dy, float* dx, int64_t M, int64_t N, int64_t K, int64_t qGroup) {
    if (!g) return DGM_ERR_ARG;
    dgm_GemmP p;
    int rc = make_p(g, "gemmDX", M, N, K, 0, qGroup, &p);
    if (rc) return rc;
    switch (bits) {
        case 32: return dgm_gemm_dx_f32(g, w, dy, dx, &p);
        case 8: return dgm_gemm_dx_i8(g, static_cast<const int8_t*>(q), scale, dy, dx, &p);
        case 4: return dgm_gemm_dx_i4(g, static_cast<const uint8_t*>(q), scale, dy, dx, &p);
        default: return dgm::fail(g, DGM_ERR_BITS, "gemmDX: unsupported bits %lld", (long long)bits);
    }
}

int dgm_gemmDW(dgm_gpu* g, const float* dy, const float* x, float* dw, int64_t M, int64_t N,
               int64_t K) {
    if (!g) return DGM_ERR_ARG;
    dgm_GemmP p;
    int rc = make_p(g, "gemmDW", M, N, K, 0, 8, &p);   // defaultQGroup, unused (GPU.swift:263)
    if (rc) return rc;
    return dgm_gemm_dw(g, dy, x, dw, &p);
}

int dgm_gemmDWAcc(dgm_gpu* g, const float* dy, const float* x, float* dw, int64_t M, int64_t N,
                  int64_t K) {
    if (!g) return DGM_ERR_ARG;
    dgm_GemmP p;
    int rc = make_p(g, "gemmDWAcc", M, N, K, 0, 8, &p);
    if (rc) return rc;
    return dgm_gemm_dw_acc(g, dy, x, dw, &p);
}

int dgm_gemmBwd(dgm_gpu* g, int64_t bits, const float* w, const void* q, const float* scale, const float* dy,
                const float* x, float* dx, float* dw, int64_t M, int64_t N, int64_t K, int64_t qGroup,
                int accumulate) {
    // GPU.gemmDW (or gemmDWAcc) then GPU.gemmDX on the same dY, as the
    // reference's backward issues them (src/GPT.swift:374-376, 384-420).
    if (!g) return DGM_ERR_ARG;
    if (bits != 32 && bits != 8 && bits != 4)
        return dgm::fail(g, DGM_ERR_BITS, "gemmBwd: unsupported bits %lld", (long long)bits);
    dgm_GemmP p;
    int rc = make_p(g, "gemmBwd", M, N, K, 0, qGroup, &p);
    if (rc) return rc;
    const char* name = bits == 32 ? "gemm_bwd_f32" : (bits == 8 ? "gemm_bwd_i8" : "gemm_bwd_i4");
    rc = dgm::enter(g, name);
    if (rc) return rc;
    rc = dgm::gemm_check_sizes(g, name, &p, int(bits));
    if (rc) return rc;
    const void* wt = bits == 32 ? static_cast<const void*>(w) : q;
    if (p.M > 0 && p.N > 0 && p.K > 0) {
        if (!dx || !dw || !dy || !x || !wt || (bits != 32 && !scale))
            return dgm::fail(g, DGM_ERR_ARG, "gemmBwd: null buffer");
        bool fused = false;
        rc = dgm::gemm_f32_bwd_pair(g, int(bits), wt, scale, dy, x, dx, dw, &p, accumulate != 0, &fused);
        if (rc) return rc;
        if (fused) {
            DGM_LAUNCH_CHECK(g, name);
            return DGM_OK;
        }
    }
    rc = accumulate ? dgm_gemm_dw_acc(g, dy, x, dw, &p) : dgm_gemm_dw(g, dy, x, dw, &p);
    if (rc) return rc;
    switch (bits) {
        case 32: return dgm_gemm_dx_f32(g, w, dy, dx, &p);
        case 8: return dgm_gemm_dx_i8(g, static_cast<const int8_t*>(q), scale, dy, dx, &p);
        default: return dgm_gemm_dx_i4(g, static_cast<const uint8_t*>(q), scale, dy, dx, &p);
    }
}

}  // extern "C"

namespace dgm {

int gemm_bwd_swiglu(dgm_gpu* g, int bits, const float* w, const void* q, const float* scale, const float* dy,
                    const float* x, const float* gate, const float* up, float* dgu, float* dw, int64_t M, int64_t N,
                    int64_t K, int64_t qGroup) {
    if (!g) return DGM_ERR_ARG;
    if (bits != 32 && bits != 8 && bits != 4)
        return fail(g, DGM_ERR_BITS, "gemmBwd: unsupported bits %d", bits);
    dgm_GemmP p;
    int rc = make_p(g, "gemmBwd", M, N, K, 0, qGroup, &p);
    if (rc) return rc;
    const char* name = bits == 32 ? "gemm_bwd_f32" : (bits == 8 ? "gemm_bwd_i8" : "gemm_bwd_i4");
    rc = gemm_check_sizes(g, name, &p, bits);
    if (rc) return rc;
    const void* wt = bits == 32 ? static_cast<const void*>(w) : q;
    if (p.M == 0 || p.N == 0 || p.K == 0) return kNotFused;
    if (!dgu || !dw || !dy || !x || !wt || !gate || !up || (bits != 32 && !scale))
        return fail(g, DGM_ERR_ARG, "gemmBwd: null buffer");
    rc = enter(g, name);
    if (rc) return rc;
    bool fused = false;
    rc = gemm_f32_bwd_pair(g, bits, wt, scale, dy, x, dgu, dw, &p, true, &fused, gate, up);
    if (rc) return rc;
    if (!fused) return kNotFused;
    DGM_LAUNCH_CHECK(g, name);
    return DGM_OK;
}

}  // namespace dgm
