// fp32-accurate GEMMs of the quantized linear path on gfx950:
//   forward  Y[m,n]  = sum_k X[m,k] * deq(W)[n,k] (+ bias[n])   (kernels.metal:128-209)
//   STE dX   dX[m,k] = sum_n dY[m,n] * deq(W)[n,k]              (kernels.metal:211-268)
//   STE dW   dW[n,k] (=|+=) sum_m dY[m,n] * X[m,k]              (kernels.metal:270-283, 1014-1027)
// deq(W)[n,k] = code[n,k] * S[n, k/G] rounded once to fp32 (the reference's
// dequant, Check.swift:433-458), or the fp32 master itself for bits = 32.
//
// Design (CDNA4, wave64): products are formed by v_mfma_f32_16x16x4_f32, so
// operands and accumulation stay fp32. Each lane fetches its MFMA operands
// straight from global memory into registers (no LDS staging): for a chunk of
// 16 contraction indices, lane (r = lane%16, q = lane/16) loads the 4
// consecutive indices 4q..4q+3, and MFMA step s consumes index 4q+s. Because
// A and B use the same permutation of the contraction index the sum is
// unchanged. A workgroup = 4 waves that split the contraction 4 ways
// (interleaved 16-wide chunks) and reduce their partial tiles through LDS in a
// fixed order, so results are deterministic. Loads of the next chunk are
// issued before the MFMAs of the current one (two-stage register pipeline).
// These shapes (the DiT linears) are latency-bound, so the design keeps many
// independent loads in flight per wave and many small workgroups.
#include "common.hpp"

namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kThreads = 256;
constexpr int MODE_FWD = 0, MODE_DX = 1, MODE_DW = 2;

struct GemmArgs {
    const float* A;       // FWD: X[M,K]; DX: dY[M,N]; DW: dY[M,N]
    const void* B;        // FWD/DX: W (fp32 master or codes); DW: X[M,K]
    const float* scale;   // S[N, K/G] (quantized W only)
    const float* bias;    // FWD only, when has_bias
    float* out;
    int rows, cols, red;  // output tile space (i, j) and contraction length
    int M, N, K;          // original GEMM sizes (leading dimensions)
    int G, groups;
    int has_bias;
    int accumulate;       // DW: += instead of =
};

template <int BITS>
__device__ __forceinline__ int code_at(const void* W, size_t idx) {
    if constexpr (BITS == 8) {
        return static_cast<const int8_t*>(W)[idx];
    } else {
        uint8_t b = static_cast<const uint8_t*>(W)[idx >> 1];
        int nib = (idx & 1) ? (b >> 4) : (b & 0xF);
        return nib >= 8 ? nib - 16 : nib;
    }
}

template <int BITS>
__device__ __forceinline__ float deq(const GemmArgs& a, int n, int k) {
    const size_t idx = size_t(n) * a.K + k;
    if constexpr (BITS == 32) {
        return static_cast<const float*>(a.B)[idx];
    } else {
        return float(code_at<BITS>(a.B, idx)) * a.scale[size_t(n) * a.groups + k / a.G];
    }
}

// A operand: 4 values A(i, c0 + s), s = 0..3; zero outside the matrix.
template <int MODE, bool VEC>
__device__ __forceinline__ void load_a(const GemmArgs& a, int i, int c0, float (&v)[4]) {
    if constexpr (MODE == MODE_FWD || MODE == MODE_DX) {
        // FWD: X[i, c] (ld K); DX: dY[i, c] (ld N). Contraction is contiguous.
        const int ld = MODE == MODE_FWD ? a.K : a.N;
        const float* row = a.A + size_t(i) * ld;
        if constexpr (VEC) {
            if (i < a.rows && c0 < a.red) {
                float4 q = *reinterpret_cast<const float4*>(row + c0);
                v[0] = q.x; v[1] = q.y; v[2] = q.z; v[3] = q.w;
            } else {
                v[0] = v[1] = v[2] = v[3] = 0.0f;
            }
        } else {
#pragma unroll
            for (int s = 0; s < 4; ++s)
                v[s] = (i < a.rows && c0 + s < a.red) ? row[c0 + s] : 0.0f;
        }
    } else {
        // DW: A(i = n, c = m) = dY[m, n]; rows of dY are strided by N.
#pragma unroll
        for (int s = 0; s < 4; ++s)
            v[s] = (i < a.rows && c0 + s < a.red) ? a.A[size_t(c0 + s) * a.N + i] : 0.0f;
    }
}

// B operand: 4 values B(c0 + s, j), s = 0..3; zero outside the matrix.
template <int MODE, int BITS, bool VEC>
__device__ __forceinline__ void load_b(const GemmArgs& a, int c0, int j, float (&v)[4]) {
    if constexpr (MODE == MODE_FWD) {
        // B(c = k, j = n) = deq(W)[n, k]: contiguous along k.
        const bool ok = j < a.cols && c0 < a.red;
        if constexpr (VEC) {
            if (!ok) {
                v[0] = v[1] = v[2] = v[3] = 0.0f;
                return;
            }
            const size_t idx = size_t(j) * a.K + c0;
            if constexpr (BITS == 32) {
                float4 q = *reinterpret_cast<const float4*>(static_cast<const float*>(a.B) + idx);
                v[0] = q.x; v[1] = q.y; v[2] = q.z; v[3] = q.w;
            } else {
                int c[4];
                if constexpr (BITS == 8) {
                    const uint32_t w = *reinterpret_cast<const uint32_t*>(static_cast<const int8_t*>(a.B) + idx);
#pragma unroll
                    for (int s = 0; s < 4; ++s) c[s] = int(int8_t((w >> (8 * s)) & 0xFF));
                } else {
                    const uint32_t w = *reinterpret_cast<const uint16_t*>(static_cast<const uint8_t*>(a.B) + (idx >> 1));
#pragma unroll
                    for (int s = 0; s < 4; ++s) {
                        int nib = int((w >> (4 * s)) & 0xF);
                        c[s] = nib >= 8 ? nib - 16 : nib;
                    }
                }
                const float* srow = a.scale + size_t(j) * a.groups;
                if ((a.G & 3) == 0) {
                    const float sc = srow[c0 / a.G];
#pragma unroll
                    for (int s = 0; s < 4; ++s) v[s] = float(c[s]) * sc;
                } else {
#pragma unroll
                    for (int s = 0; s < 4; ++s) v[s] = float(c[s]) * srow[(c0 + s) / a.G];
                }
            }
        } else {
#pragma unroll
            for (int s = 0; s < 4; ++s)
                v[s] = (j < a.cols && c0 + s < a.red) ? deq<BITS>(a, j, c0 + s) : 0.0f;
        }
    } else if constexpr (MODE == MODE_DX) {
        // B(c = n, j = k) = deq(W)[n, k]: rows strided by K.
#pragma unroll
        for (int s = 0; s < 4; ++s)
            v[s] = (j < a.cols && c0 + s < a.red) ? deq<BITS>(a, c0 + s, j) : 0.0f;
    } else {
        // DW: B(c = m, j = k) = X[m, k].
        const float* X = static_cast<const float*>(a.B);
#pragma unroll
        for (int s = 0; s < 4; ++s)
            v[s] = (j < a.cols && c0 + s < a.red) ? X[size_t(c0 + s) * a.K + j] : 0.0f;
    }
}

template <int MODE, int BITS, int TM, int TN, bool VEC>
__global__ __launch_bounds__(kThreads) void gemm_f32_kernel(GemmArgs a) {
    constexpr int RT = TM / 16, CT = TN / 16;
    __shared__ float part[4][TM * TN];

    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int r16 = lane & 15;
    const int q4 = lane >> 4;
    const int i0 = blockIdx.y * TM;
    const int j0 = blockIdx.x * TN;

    f32x4 acc[RT][CT];
#pragma unroll
    for (int ti = 0; ti < RT; ++ti)
#pragma unroll
        for (int tj = 0; tj < CT; ++tj) acc[ti][tj] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

    const int nchunks = (a.red + 15) / 16;
    float av[2][RT][4], bv[2][CT][4];

    auto fetch = [&](int stage, int ch) {
        const int c0 = ch * 16 + 4 * q4;
#pragma unroll
        for (int ti = 0; ti < RT; ++ti) load_a<MODE, VEC>(a, i0 + ti * 16 + r16, c0, av[stage][ti]);
#pragma unroll
        for (int tj = 0; tj < CT; ++tj) load_b<MODE, BITS, VEC>(a, c0, j0 + tj * 16 + r16, bv[stage][tj]);
    };
    auto compute = [&](int stage) {
#pragma unroll
        for (int s = 0; s < 4; ++s)
#pragma unroll
            for (int ti = 0; ti < RT; ++ti)
#pragma unroll
                for (int tj = 0; tj < CT; ++tj)
                    acc[ti][tj] = __builtin_amdgcn_mfma_f32_16x16x4f32(av[stage][ti][s], bv[stage][tj][s],
                                                                      acc[ti][tj], 0, 0, 0);
    };

    int ch = wave;
    if (ch < nchunks) fetch(0, ch);
    while (ch < nchunks) {
        const int nxt = ch + 4;
        if (nxt < nchunks) fetch(1, nxt);
        compute(0);
        if (nxt >= nchunks) break;
        const int nxt2 = nxt + 4;
        if (nxt2 < nchunks) fetch(0, nxt2);
        compute(1);
        ch = nxt2;
    }

    // D layout of 16x16x4 f32: lane holds rows 4*(lane/16) + r, column lane%16.
#pragma unroll
    for (int ti = 0; ti < RT; ++ti)
#pragma unroll
        for (int tj = 0; tj < CT; ++tj)
#pragma unroll
            for (int r = 0; r < 4; ++r)
                part[wave][(ti * 16 + 4 * q4 + r) * TN + tj * 16 + r16] = acc[ti][tj][r];
    __syncthreads();

    for (int e = threadIdx.x; e < TM * TN; e += kThreads) {
        const int i = i0 + e / TN;
        const int j = j0 + e % TN;
        if (i >= a.rows || j >= a.cols) continue;
        float v = part[0][e];
        v += part[1][e];
        v += part[2][e];
        v += part[3][e];
        float* o = a.out + size_t(i) * a.cols + j;
        if constexpr (MODE == MODE_FWD) {
            if (a.has_bias) v += a.bias[j];
            *o = v;
        } else if constexpr (MODE == MODE_DW) {
            if (a.accumulate) *o += v;
            else *o = v;
        } else {
            *o = v;
        }
    }
}

template <int MODE, int BITS, int TM, int TN>
void launch_tile(const GemmArgs& a, bool vec, hipStream_t st) {
    dim3 grid(dgm::ceil_div(a.cols, TN), dgm::ceil_div(a.rows, TM));
    if (vec)
        hipLaunchKernelGGL((gemm_f32_kernel<MODE, BITS, TM, TN, true>), grid, dim3(kThreads), 0, st, a);
    else
        hipLaunchKernelGGL((gemm_f32_kernel<MODE, BITS, TM, TN, false>), grid, dim3(kThreads), 0, st, a);
}

template <int MODE, int BITS>
void launch_gemm(const GemmArgs& a, bool vec, int num_cus, hipStream_t st) {
    // Pick the largest tile that still gives every CU a couple of workgroups.
    const int64_t t32 = int64_t(dgm::ceil_div(a.rows, 32)) * dgm::ceil_div(a.cols, 32);
    const int64_t t16x32 = int64_t(dgm::ceil_div(a.rows, 16)) * dgm::ceil_div(a.cols, 32);
    if (t32 >= 2 * num_cus)
        launch_tile<MODE, BITS, 32, 32>(a, vec, st);
    else if (t16x32 >= 2 * num_cus)
        launch_tile<MODE, BITS, 16, 32>(a, vec, st);
    else
        launch_tile<MODE, BITS, 16, 16>(a, vec, st);
}

int check_sizes(dgm_gpu* g, const char* name, const dgm_GemmP* p, int bits) {
    if (!p) return dgm::fail(g, DGM_ERR_ARG, "%s: null GemmP", name);
    if (int64_t(p->M) > dgm::kMaxIndex || int64_t(p->N) > dgm::kMaxIndex ||
        int64_t(p->K) > dgm::kMaxIndex)
        return dgm::fail(g, DGM_ERR_UNSUPPORTED, "%s: size beyond 2^31", name);
    if (int64_t(p->M) * p->K > (int64_t(1) << 40) || int64_t(p->N) * p->K > (int64_t(1) << 40))
        return dgm::fail(g, DGM_ERR_UNSUPPORTED, "%s: matrix too large", name);
    if (bits != 32) {
        // src/GPU.swift:229,247 and src/Params.swift:168-172.
        if (p->qGroup == 0 || p->K % p->qGroup != 0)
            return dgm::fail(g, DGM_ERR_SHAPE, "%s: K=%u not divisible by group %u", name, p->K,
                             p->qGroup);
        if (bits == 4 && (p->qGroup % 2) != 0)
            return dgm::fail(g, DGM_ERR_SHAPE, "%s: quant group must be even for int4", name);
    }
    return DGM_OK;
}

}  // namespace

namespace dgm {

bool skinny_ok(int bits, const void* W, const float* X, const dgm_GemmP* p);
int skinny_fwd(dgm_gpu* g, int bits, const void* W, const float* scale, const float* X,
               const float* bias, float* Y, const dgm_GemmP* p);
bool bf16_ok(int bits, const void* W, const float* X, const float* S, const dgm_GemmP* p);
int bf16_fwd(dgm_gpu* g, int bits, const void* W, const float* scale, const float* X,
             const float* bias, float* Y, const dgm_GemmP* p);

// Entry used by the dispatcher in gemm_entry.hip; declared there.
int gemm_f32_fwd(dgm_gpu* g, int bits, const void* W, const float* scale, const float* X,
                 const float* bias, float* Y, const dgm_GemmP* p) {
    // Decode-shaped quantized forwards stream W once through int8 MFMA.
    if (skinny_ok(bits, W, X, p)) return skinny_fwd(g, bits, W, scale, X, bias, Y, p);
    // Larger M in the reduced-precision mode: bf16 MFMA with W dequantized in LDS.
    if (g->math == DGM_MATH_BF16 && bf16_ok(bits, W, X, scale, p))
        return bf16_fwd(g, bits, W, scale, X, bias, Y, p);
    GemmArgs a{};
    a.A = X; a.B = W; a.scale = scale; a.bias = bias; a.out = Y;
    a.M = p->M; a.N = p->N; a.K = p->K;
    a.rows = p->M; a.cols = p->N; a.red = p->K;
    a.G = bits == 32 ? 1 : int(p->qGroup);
    a.groups = bits == 32 ? 0 : int(p->K / p->qGroup);
    a.has_bias = p->hasBias != 0;
    const size_t wal = bits == 32 ? 16 : (bits == 8 ? 4 : 2);
    const bool vec = (p->K % 4) == 0 && aligned(X, 16) && aligned(W, wal);
    if (bits == 32) launch_gemm<MODE_FWD, 32>(a, vec, g->num_cus, g->stream);
    else if (bits == 8) launch_gemm<MODE_FWD, 8>(a, vec, g->num_cus, g->stream);
    else launch_gemm<MODE_FWD, 4>(a, vec, g->num_cus, g->stream);
    return DGM_OK;
}

int gemm_f32_dx(dgm_gpu* g, int bits, const void* W, const float* scale, const float* dY,
                float* dX, const dgm_GemmP* p) {
    GemmArgs a{};
    a.A = dY; a.B = W; a.scale = scale; a.out = dX;
    a.M = p->M; a.N = p->N; a.K = p->K;
    a.rows = p->M; a.cols = p->K; a.red = p->N;
    a.G = bits == 32 ? 1 : int(p->qGroup);
    a.groups = bits == 32 ? 0 : int(p->K / p->qGroup);
    const bool vec = (p->N % 4) == 0 && aligned(dY, 16);
    if (bits == 32) launch_gemm<MODE_DX, 32>(a, vec, g->num_cus, g->stream);
    else if (bits == 8) launch_gemm<MODE_DX, 8>(a, vec, g->num_cus, g->stream);
    else launch_gemm<MODE_DX, 4>(a, vec, g->num_cus, g->stream);
    return DGM_OK;
}

int gemm_f32_dw(dgm_gpu* g, const float* dY, const float* X, float* dW, const dgm_GemmP* p,
                bool accumulate) {
    GemmArgs a{};
    a.A = dY; a.B = X; a.out = dW;
    a.M = p->M; a.N = p->N; a.K = p->K;
    a.rows = p->N; a.cols = p->K; a.red = p->M;
    a.G = 1; a.groups = 0;
    a.accumulate = accumulate;
    launch_gemm<MODE_DW, 32>(a, false, g->num_cus, g->stream);
    return DGM_OK;
}

int gemm_check_sizes(dgm_gpu* g, const char* name, const dgm_GemmP* p, int bits) {
    return check_sizes(g, name, p, bits);
}

}  // namespace dgm
