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
#include "dw_tile.hpp"

namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(1))) const void global_cvoid;
typedef __attribute__((address_space(3))) void lds_void;

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
    // DX (LDS kernel) only, when set: out gets [rows, 2K] rows [dgate | dup],
    // the SwiGLU backward of dX against gate / up [rows, K].
    const float* sg_gate;
    const float* sg_up;
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

// ---- deep-prefetch variant ---------------------------------------------------
// Same products and the same per-wave split into partial tiles, but each wave
// owns a CONTIGUOUS run of 16-wide contraction chunks and issues the raw loads
// of up to PF chunks (activations, codes, scales) before converting any of
// them, so a wave waits for one memory latency per PF chunks instead of one
// per chunk. Loads are never predicated: row/column indices past the matrix
// are clamped (their results land in rows/columns that are not stored) and the
// contraction length is a multiple of 16. Workgroups are numbered XCD-aware:
// consecutive tiles sharing an operand strip (rows of X or dY for the
// forward/dX, columns of X for dW) run on one XCD, so that strip is fetched
// into one L2 instead of eight.
// Body of one tile; `blk` is the workgroup's index within its own grid, part
// 4 * TM * TN floats of LDS.
template <int MODE, int BITS, int TM, int TN, int PF>
__device__ __forceinline__ void deep_tile(const GemmArgs& a, int tiles_i, int tiles_j, int per_xcd, int blk,
                                          float (*part)[TM * TN]) {
    constexpr int RT = TM / 16, CT = TN / 16;
    const int t = (blk & 7) * per_xcd + (blk >> 3);
    if (t >= tiles_i * tiles_j) return;
    int ti, tj;
    if constexpr (MODE == MODE_DW) {
        tj = t / tiles_i;
        ti = t - tj * tiles_i;
    } else {
        ti = t / tiles_j;
        tj = t - ti * tiles_j;
    }
    const int i0 = ti * TM, j0 = tj * TN;
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int r16 = lane & 15;
    const int q4 = lane >> 4;

    int irow[RT], jcol[CT];
#pragma unroll
    for (int x = 0; x < RT; ++x) irow[x] = min(i0 + x * 16 + r16, a.rows - 1);
#pragma unroll
    for (int y = 0; y < CT; ++y) jcol[y] = min(j0 + y * 16 + r16, a.cols - 1);

    f32x4 acc[RT][CT];
#pragma unroll
    for (int x = 0; x < RT; ++x)
#pragma unroll
        for (int y = 0; y < CT; ++y) acc[x][y] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

    const int nchunks = a.red >> 4;
    const int cpw = (nchunks + 3) >> 2;
    const int begin = wave * cpw;
    const int end = min(nchunks, begin + cpw);
    const int last = max(0, min(end, nchunks) - 1);

    float ra[PF][RT][4];
    float rb[PF][CT][4];   // fp32 operand, or codes (as int bits) for quantized W
    float rs[PF][CT][4];   // per-element scales (DX) / rs[..][0] per-lane scale (FWD)

    for (int base = begin; base < end; base += PF) {
        // -- issue every load of the round --------------------------------------
#pragma unroll
        for (int u = 0; u < PF; ++u) {
            const int ch = min(base + u, last);
            const int c0 = ch * 16 + 4 * q4;
#pragma unroll
            for (int x = 0; x < RT; ++x) {
                if constexpr (MODE == MODE_DW) {
#pragma unroll
                    for (int s = 0; s < 4; ++s) ra[u][x][s] = a.A[size_t(c0 + s) * a.N + irow[x]];
                } else {
                    const int ld = MODE == MODE_FWD ? a.K : a.N;
                    const float4 v = *reinterpret_cast<const float4*>(a.A + size_t(irow[x]) * ld + c0);
                    ra[u][x][0] = v.x; ra[u][x][1] = v.y; ra[u][x][2] = v.z; ra[u][x][3] = v.w;
                }
            }
#pragma unroll
            for (int y = 0; y < CT; ++y) {
                const int j = jcol[y];
                if constexpr (MODE == MODE_FWD) {
                    const size_t idx = size_t(j) * a.K + c0;
                    if constexpr (BITS == 32) {
                        const float4 v = *reinterpret_cast<const float4*>(static_cast<const float*>(a.B) + idx);
                        rb[u][y][0] = v.x; rb[u][y][1] = v.y; rb[u][y][2] = v.z; rb[u][y][3] = v.w;
                    } else {
                        uint32_t w;
                        if constexpr (BITS == 8)
                            w = *reinterpret_cast<const uint32_t*>(static_cast<const int8_t*>(a.B) + idx);
                        else
                            w = *reinterpret_cast<const uint16_t*>(static_cast<const uint8_t*>(a.B) + (idx >> 1));
                        rb[u][y][0] = __uint_as_float(w);
                        rs[u][y][0] = a.scale[size_t(j) * a.groups + c0 / a.G];
                    }
                } else if constexpr (MODE == MODE_DX) {
#pragma unroll
                    for (int s = 0; s < 4; ++s) {
                        const size_t idx = size_t(c0 + s) * a.K + j;
                        if constexpr (BITS == 32) {
                            rb[u][y][s] = static_cast<const float*>(a.B)[idx];
                        } else {
                            const uint32_t w = BITS == 8 ? uint32_t(static_cast<const uint8_t*>(a.B)[idx])
                                                         : uint32_t(static_cast<const uint8_t*>(a.B)[idx >> 1]);
                            rb[u][y][s] = __uint_as_float(w);
                            rs[u][y][s] = a.scale[size_t(c0 + s) * a.groups + j / a.G];
                        }
                    }
                } else {
                    const float* X = static_cast<const float*>(a.B);
#pragma unroll
                    for (int s = 0; s < 4; ++s) rb[u][y][s] = X[size_t(c0 + s) * a.K + j];
                }
            }
        }
        __builtin_amdgcn_sched_barrier(0);
        // -- convert and multiply, chunk by chunk in issue order ------------------
#pragma unroll
        for (int u = 0; u < PF; ++u) {
            if (base + u >= end) continue;
            float bv[CT][4];
#pragma unroll
            for (int y = 0; y < CT; ++y) {
                if constexpr (BITS == 32) {
#pragma unroll
                    for (int s = 0; s < 4; ++s) bv[y][s] = rb[u][y][s];
                } else if constexpr (MODE == MODE_FWD) {
                    const uint32_t w = __float_as_uint(rb[u][y][0]);
#pragma unroll
                    for (int s = 0; s < 4; ++s) {
                        int c;
                        if constexpr (BITS == 8) {
                            c = int(int8_t((w >> (8 * s)) & 0xFF));
                        } else {
                            const int nib = int((w >> (4 * s)) & 0xF);
                            c = nib >= 8 ? nib - 16 : nib;
                        }
                        bv[y][s] = float(c) * rs[u][y][0];
                    }
                } else {
                    // DX: element s is row n = c0 + s of W at column j.
#pragma unroll
                    for (int s = 0; s < 4; ++s) {
                        const uint32_t w = __float_as_uint(rb[u][y][s]);
                        int c;
                        if constexpr (BITS == 8) {
                            c = int(int8_t(w & 0xFF));
                        } else {
                            const int nib = int((jcol[y] & 1) ? (w >> 4) : (w & 0xF));
                            c = nib >= 8 ? nib - 16 : nib;
                        }
                        bv[y][s] = float(c) * rs[u][y][s];
                    }
                }
            }
#pragma unroll
            for (int s = 0; s < 4; ++s)
#pragma unroll
                for (int x = 0; x < RT; ++x)
#pragma unroll
                    for (int y = 0; y < CT; ++y)
                        acc[x][y] = __builtin_amdgcn_mfma_f32_16x16x4f32(ra[u][x][s], bv[y][s], acc[x][y], 0, 0, 0);
        }
    }

#pragma unroll
    for (int x = 0; x < RT; ++x)
#pragma unroll
        for (int y = 0; y < CT; ++y)
#pragma unroll
            for (int r = 0; r < 4; ++r)
                part[wave][(x * 16 + 4 * q4 + r) * TN + y * 16 + r16] = acc[x][y][r];
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

template <int MODE, int BITS, int TM, int TN, int PF>
__global__ __launch_bounds__(kThreads) void gemm_deep_kernel(GemmArgs a, int tiles_i, int tiles_j, int per_xcd) {
    __shared__ float part[4][TM * TN];
    deep_tile<MODE, BITS, TM, TN, PF>(a, tiles_i, tiles_j, per_xcd, int(blockIdx.x), part);
}

template <int MODE, int BITS, int TM, int TN, int PF>
void launch_deep_tile(const GemmArgs& a, hipStream_t st) {
    const int ti = int(dgm::ceil_div(a.rows, TM)), tj = int(dgm::ceil_div(a.cols, TN));
    const int64_t nt = int64_t(ti) * tj;
    const int per = int((nt + 7) / 8);
    hipLaunchKernelGGL((gemm_deep_kernel<MODE, BITS, TM, TN, PF>), dim3(unsigned(per) * 8u), dim3(kThreads), 0, st,
                       a, ti, tj, per);
}

// The deep variant needs a contraction that is a multiple of 16, 16-byte
// aligned activation rows for the forward/dX, and (quantized forward) a group
// that is a multiple of 4 so each lane's 4 consecutive weights share a scale.
template <int MODE>
bool deep_ok(const GemmArgs& a, int bits, bool vec) {
    if (a.red % 16 != 0 || a.red == 0 || a.rows == 0 || a.cols == 0) return false;
    if (int64_t(a.rows) * dgm::ceil_div(a.cols, 16) > (int64_t(1) << 30)) return false;
    if (MODE == MODE_FWD) return vec && (bits == 32 || a.G % 4 == 0);
    if (MODE == MODE_DX) return vec;
    return true;
}

template <int MODE, int BITS>
void launch_deep(const GemmArgs& a, int num_cus, hipStream_t st) {
    const int64_t t32 = int64_t(dgm::ceil_div(a.rows, 32)) * dgm::ceil_div(a.cols, 32);
    const int64_t t16x32 = int64_t(dgm::ceil_div(a.rows, 16)) * dgm::ceil_div(a.cols, 32);
    if (t32 >= 2 * num_cus)
        launch_deep_tile<MODE, BITS, 32, 32, 6>(a, st);
    else if (t16x32 >= 2 * num_cus)
        launch_deep_tile<MODE, BITS, 16, 32, 8>(a, st);
    else
        launch_deep_tile<MODE, BITS, 16, 16, 12>(a, st);
}

// ---- LDS-staged forward for short contractions (K <= 1024, K % 64 == 0) -------
// The latency-bound shapes of the DiT linears. A workgroup owns 16 rows of Y
// and 16*(4/KS) columns: its 16 x K block of X is read once with fully
// coalesced 16-byte loads (each wave instruction covers 1 KB of whole rows)
// and parked in LDS; every wave then reads it back in MFMA layout. Waves are
// arranged KS (contraction parts) x 4/KS (16-column groups). Within a stage of
// 64 contraction indices, lane (r, q) multiplies indices 16q .. 16q+15 (chunk c
// of the stage uses 16q + 4c .. 16q + 4c + 3), so each lane's weight codes for
// a stage are ONE contiguous 8-byte (int4) / 16-byte (int8) load and one
// scale, instead of four 16-row gathers. X in LDS is stored with the 16-byte
// slot index XOR-ed by (row & 15): the 16 rows read by one MFMA operand fetch
// land in 16 distinct slots, free of bank conflicts. Contraction parts are
// reduced through LDS in a fixed order.
template <int BITS, int KS>
__global__ __launch_bounds__(kThreads) void gemm_fwd_lds_kernel(GemmArgs a, int tiles_i, int tiles_j, int per_xcd) {
    constexpr int NS = 4 / KS;
    constexpr int TN = 16 * NS;
    extern __shared__ __align__(16) float4 xs[];   // [16][K/4] slots, swizzled

    const int t = (blockIdx.x & 7) * per_xcd + (blockIdx.x >> 3);
    if (t >= tiles_i * tiles_j) return;
    const int ti = t / tiles_j, tj = t - ti * tiles_j;
    const int i0 = ti * 16, j0 = tj * TN;
    const int K = a.K;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int r16 = lane & 15, q4 = lane >> 4;
    const int wk = wave % KS, wn = wave / KS;
    const int nst = K >> 6;

    // -- weight codes + scales of this wave's stages (issued first; they are
    // consumed last, after X has been staged).
    constexpr int MAXST = (BITS == 32 ? 8 : 16) / KS;   // K <= 1024 (512 for fp32 weights)
    const int n = min(j0 + wn * 16 + r16, a.cols - 1);
    uint32_t wc[MAXST][BITS == 4 ? 2 : 4];
    float4 wf[MAXST][BITS == 32 ? 4 : 1];
    float sc[MAXST];
#pragma unroll
    for (int u = 0; u < MAXST; ++u) {
        const int st = wk + u * KS;
        if (st >= nst) continue;   // wave-uniform; these loads are only read after the barrier
        const int k = st * 64 + 16 * q4;
        if constexpr (BITS == 32) {
            const float4* p = reinterpret_cast<const float4*>(static_cast<const float*>(a.B) + size_t(n) * K + k);
#pragma unroll
            for (int e = 0; e < 4; ++e) wf[u][e] = p[e];
        } else if constexpr (BITS == 8) {
            const uint4 v = *reinterpret_cast<const uint4*>(static_cast<const int8_t*>(a.B) + size_t(n) * K + k);
            wc[u][0] = v.x; wc[u][1] = v.y; wc[u][2] = v.z; wc[u][3] = v.w;
            sc[u] = a.scale[size_t(n) * a.groups + k / a.G];
        } else {
            const uint2 v = *reinterpret_cast<const uint2*>(static_cast<const uint8_t*>(a.B) + ((size_t(n) * K + k) >> 1));
            wc[u][0] = v.x; wc[u][1] = v.y;
            sc[u] = a.scale[size_t(n) * a.groups + k / a.G];
        }
    }

    // -- X block: 16 rows x K floats straight into LDS (global_load_lds, 16 B
    // per lane; a wave instruction fills 1 KB of LDS in lane order). LDS slot
    // (row, pos) receives the row's global slot pos ^ (row & 15).
    const int spr = K >> 2;                   // 16-byte slots per row
    const int ninst = (16 * spr) >> 6;        // wave instructions for the block
    uint8_t* xb = reinterpret_cast<uint8_t*>(xs);
    for (int ii = wave; ii < ninst; ii += 4) {
        const int L = ii * 64 + lane;
        const int row = L / spr, pos = L - row * spr;
        const int gr = min(i0 + row, a.rows - 1);
        const float* src = a.A + size_t(gr) * K + ((pos ^ (row & 15)) << 2);
        __builtin_amdgcn_global_load_lds((global_cvoid*)src, (lds_void*)(xb + ii * 1024), 16, 0, 0);
    }
    __syncthreads();

    f32x4 acc = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int u = 0; u < MAXST; ++u) {
        const int st = wk + u * KS;
        if (st >= nst) break;
        const float4* xrow = xs + r16 * spr;
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            const float4 xv = xrow[(st * 16 + 4 * q4 + c) ^ r16];
            float bv[4];
            if constexpr (BITS == 32) {
                const float4 w = wf[u][c];
                bv[0] = w.x; bv[1] = w.y; bv[2] = w.z; bv[3] = w.w;
            } else if constexpr (BITS == 8) {
                const uint32_t w = wc[u][c];
#pragma unroll
                for (int s2 = 0; s2 < 4; ++s2) bv[s2] = float(int(int8_t((w >> (8 * s2)) & 0xFF))) * sc[u];
            } else {
                const uint32_t w = wc[u][c >> 1] >> (16 * (c & 1));
#pragma unroll
                for (int s2 = 0; s2 < 4; ++s2) bv[s2] = float(int(__builtin_amdgcn_sbfe(int(w), 4 * s2, 4))) * sc[u];
            }
            acc = __builtin_amdgcn_mfma_f32_16x16x4f32(xv.x, bv[0], acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_f32_16x16x4f32(xv.y, bv[1], acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_f32_16x16x4f32(xv.z, bv[2], acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_f32_16x16x4f32(xv.w, bv[3], acc, 0, 0, 0);
        }
    }

    // -- reduce contraction parts in order and store. acc: rows 4*q4 + r, column r16.
    // The bias is added before the first store: a load whose value only the
    // conditional stores use makes the compiler wait for every outstanding
    // memory operation, the earlier stores included, before each store.
    if constexpr (KS == 1) {
        const int j = j0 + wn * 16 + r16;
        if (j < a.cols) {
            if (a.has_bias) acc += a.bias[j];
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int i = i0 + 4 * q4 + r;
                if (i < a.rows) a.out[size_t(i) * a.cols + j] = acc[r];
            }
        }
    } else {
        __syncthreads();   // X no longer read: reuse LDS for the partial tiles
        float* part = reinterpret_cast<float*>(xs);   // [KS][16][TN]
#pragma unroll
        for (int r = 0; r < 4; ++r) part[(wk * 16 + 4 * q4 + r) * TN + wn * 16 + r16] = acc[r];
        __syncthreads();
        static_assert(kThreads % TN == 0, "a thread keeps one column");
        const int j = j0 + threadIdx.x % TN;
        if (j >= a.cols) return;
        float bb = a.has_bias ? a.bias[j] : 0.0f;
        asm volatile("" : "+v"(bb));
        for (int e = threadIdx.x; e < 16 * TN; e += kThreads) {
            const int i = i0 + e / TN;
            if (i >= a.rows) break;
            float v = part[e];
#pragma unroll
            for (int p2 = 1; p2 < KS; ++p2) v += part[p2 * 16 * TN + e];
            if (a.has_bias) v += bb;
            a.out[size_t(i) * a.cols + j] = v;
        }
    }
}

template <int BITS, int KS>
void launch_fwd_lds_ks(const GemmArgs& a, hipStream_t st) {
    constexpr int TN = 16 * (4 / KS);
    const int ti = int(dgm::ceil_div(a.rows, 16)), tj = int(dgm::ceil_div(a.cols, TN));
    const int64_t nt = int64_t(ti) * tj;
    const int per = int((nt + 7) / 8);
    const size_t lds = size_t(16) * a.K * sizeof(float);
    hipLaunchKernelGGL((gemm_fwd_lds_kernel<BITS, KS>), dim3(unsigned(per) * 8u), dim3(kThreads), lds, st, a, ti, tj,
                       per);
}

// The 4-way contraction split (16 x 16 tiles) with X read straight into
// registers. With one 16-column group per workgroup no two waves read the same
// X element, so the LDS block and the barrier before the first MFMA are pure
// latency: here every lane loads, for each of its stages, the 64 contiguous
// bytes of X row r16 that it multiplies (indices 16q .. 16q+15 of the stage)
// as four 16-byte loads, right after that stage's weight codes. Stage u's
// MFMAs wait only for the loads issued up to stage u (in-order vmcnt), so the
// first products start while later stages are still in flight. SPW = stages
// per wave = K / 256 exactly: the body is one basic block, so the compiler
// cannot sink a stage's loads down to its products. The arithmetic, the order
// of the sums and the fixed-order reduction of the 4 parts are those of
// gemm_fwd_lds_kernel<BITS, 4>, so the two give bitwise equal results.
template <int BITS, int SPW>
__global__ __launch_bounds__(kThreads) void gemm_fwd_reg_kernel(GemmArgs a, int tiles_i, int tiles_j, int per_xcd) {
    __shared__ float part[4 * 16 * 16];
    const int t = (blockIdx.x & 7) * per_xcd + (blockIdx.x >> 3);
    if (t >= tiles_i * tiles_j) return;
    const int ti = t / tiles_j, tj = t - ti * tiles_j;
    const int i0 = ti * 16, j0 = tj * 16;
    const int K = a.K;   // == 256 * SPW
    const int lane = threadIdx.x & 63, wk = threadIdx.x >> 6;
    const int r16 = lane & 15, q4 = lane >> 4;
    const int n = min(j0 + r16, a.cols - 1);
    const float* xr = a.A + size_t(min(i0 + r16, a.rows - 1)) * K + 16 * q4;

    uint32_t wc[SPW][BITS == 4 ? 2 : 4];
    float4 wf[SPW][BITS == 32 ? 4 : 1];
    float sc[SPW];
    float4 xv[SPW][4];
#pragma unroll
    for (int u = 0; u < SPW; ++u) {
        const int st = wk + 4 * u;
        const int k = st * 64 + 16 * q4;
        if constexpr (BITS == 32) {
            const float4* p = reinterpret_cast<const float4*>(static_cast<const float*>(a.B) + size_t(n) * K + k);
#pragma unroll
            for (int e = 0; e < 4; ++e) wf[u][e] = p[e];
        } else if constexpr (BITS == 8) {
            const uint4 v = *reinterpret_cast<const uint4*>(static_cast<const int8_t*>(a.B) + size_t(n) * K + k);
            wc[u][0] = v.x; wc[u][1] = v.y; wc[u][2] = v.z; wc[u][3] = v.w;
            sc[u] = a.scale[size_t(n) * a.groups + k / a.G];
        } else {
            const uint2 v = *reinterpret_cast<const uint2*>(static_cast<const uint8_t*>(a.B) + ((size_t(n) * K + k) >> 1));
            wc[u][0] = v.x; wc[u][1] = v.y;
            sc[u] = a.scale[size_t(n) * a.groups + k / a.G];
        }
        const float4* xp = reinterpret_cast<const float4*>(xr + st * 64);
#pragma unroll
        for (int c = 0; c < 4; ++c) xv[u][c] = xp[c];
    }
    // This thread's output element after the reduction, and its bias.
    const int e = threadIdx.x;   // 256 threads = the 16 x 16 tile
    const int i = i0 + (e >> 4), j = j0 + (e & 15);
    const float bb = a.has_bias ? a.bias[min(j, a.cols - 1)] : 0.0f;
    // Keep every load above the first wait: left alone, the scheduler moves the
    // later stages' loads between the MFMAs, after the wait for stage 0, which
    // exposes a second memory latency.
    __builtin_amdgcn_sched_barrier(0);

    f32x4 acc = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int u = 0; u < SPW; ++u) {
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            const float4 x = xv[u][c];
            float bv[4];
            if constexpr (BITS == 32) {
                const float4 w = wf[u][c];
                bv[0] = w.x; bv[1] = w.y; bv[2] = w.z; bv[3] = w.w;
            } else if constexpr (BITS == 8) {
                const uint32_t w = wc[u][c];
#pragma unroll
                for (int s2 = 0; s2 < 4; ++s2) bv[s2] = float(int(int8_t((w >> (8 * s2)) & 0xFF))) * sc[u];
            } else {
                const uint32_t w = wc[u][c >> 1] >> (16 * (c & 1));
#pragma unroll
                for (int s2 = 0; s2 < 4; ++s2) bv[s2] = float(int(__builtin_amdgcn_sbfe(int(w), 4 * s2, 4))) * sc[u];
            }
            acc = __builtin_amdgcn_mfma_f32_16x16x4f32(x.x, bv[0], acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_f32_16x16x4f32(x.y, bv[1], acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_f32_16x16x4f32(x.z, bv[2], acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_f32_16x16x4f32(x.w, bv[3], acc, 0, 0, 0);
        }
    }

    // acc: rows 4*q4 + r, column r16. Parts summed in order 0..3, then the bias.
#pragma unroll
    for (int r = 0; r < 4; ++r) part[(wk * 16 + 4 * q4 + r) * 16 + r16] = acc[r];
    __syncthreads();
    if (i < a.rows && j < a.cols) {
        float v = part[e];
#pragma unroll
        for (int p2 = 1; p2 < 4; ++p2) v += part[p2 * 256 + e];
        if (a.has_bias) v += bb;
        a.out[size_t(i) * a.cols + j] = v;
    }
}

template <int BITS, int SPW>
void launch_fwd_reg_spw(const GemmArgs& a, hipStream_t st) {
    const int ti = int(dgm::ceil_div(a.rows, 16)), tj = int(dgm::ceil_div(a.cols, 16));
    const int per = int((int64_t(ti) * tj + 7) / 8);
    hipLaunchKernelGGL((gemm_fwd_reg_kernel<BITS, SPW>), dim3(unsigned(per) * 8u), dim3(kThreads), 0, st, a, ti, tj,
                       per);
}

// K % 256 == 0 (checked by the caller); K <= 1024, 512 for fp32 weights.
template <int BITS>
void launch_fwd_reg(const GemmArgs& a, hipStream_t st) {
    const int spw = a.K / 256;
    if constexpr (BITS == 32) {
        if (spw == 1) launch_fwd_reg_spw<BITS, 1>(a, st);
        else launch_fwd_reg_spw<BITS, 2>(a, st);
    } else {
        if (spw == 1) launch_fwd_reg_spw<BITS, 1>(a, st);
        else if (spw == 2) launch_fwd_reg_spw<BITS, 2>(a, st);
        else if (spw == 3) launch_fwd_reg_spw<BITS, 3>(a, st);
        else launch_fwd_reg_spw<BITS, 4>(a, st);
    }
}

// ---- Pipelined forward for quantized weights: 16 x 32 tiles, 8 waves ----------
// Measured on these latency-bound shapes, a CU pulls data from L2 at only
// ~27 B/ns (outstanding misses x L2 latency), so what matters is the bytes each
// CU must receive and how early the MFMAs can start. A workgroup owns 16 rows x
// 32 columns of Y; its 8 waves are 4 contraction parts (wk: stages wk, wk+4,
// ...) x 2 column groups (wn). Everything it reads is moved into LDS by
// direct-to-LDS loads whose 64 lanes cover whole cache lines: first the W codes
// of the 32 columns (one contiguous chunk of 32 rows) and their scales (one
// contiguous chunk of 32 x groups floats), then X stage by stage (16 rows x 64
// floats = 4 KB per stage, stored stage-major, each of the two waves of a
// contraction part loading 8 of the rows). Before stage u a wave waits only for
// its own loads up to that stage (vmcnt in issue order) and meets the others at
// a barrier, so the MFMAs of early stages overlap the loads of later ones.
// The LDS reads are inline asm: the compiler cannot tell them apart from the
// pending direct-to-LDS loads and would otherwise wait for all of them before
// the first read. Swizzles: X slot p of row r is stored at p ^ r; W slot p of
// row r at p ^ f(r), f chosen from the row stride so that the 16 rows read by
// one operand fetch fall in distinct banks. Products, their order and the
// fixed-order reduction of the 4 parts are those of gemm_fwd_lds_kernel<BITS, 4>:
// the results are bitwise equal.
__device__ __forceinline__ uint32_t lds_off(const void* p) {
    return uint32_t(reinterpret_cast<uintptr_t>((const __attribute__((address_space(3))) char*)(p)));
}

template <int VM>
__device__ __forceinline__ void wait_own_loads_and_barrier() {
    asm volatile("s_waitcnt vmcnt(%0)\n\ts_barrier" ::"n"(VM) : "memory");
}

__device__ __forceinline__ void lds_read_x4(float4& x0, float4& x1, float4& x2, float4& x3, uint32_t a0, uint32_t a1,
                                            uint32_t a2, uint32_t a3) {
    asm volatile(
        "ds_read_b128 %0, %4\n\t"
        "ds_read_b128 %1, %5\n\t"
        "ds_read_b128 %2, %6\n\t"
        "ds_read_b128 %3, %7\n\t"
        "s_waitcnt lgkmcnt(0)"
        : "=&v"(x0), "=&v"(x1), "=&v"(x2), "=&v"(x3)
        : "v"(a0), "v"(a1), "v"(a2), "v"(a3)
        : "memory");
}

// One stage's codes (8 bytes int4 / 16 bytes int8) and scale of a lane.
template <int BITS>
__device__ __forceinline__ void lds_read_codes(uint32_t (&w)[BITS == 4 ? 2 : 4], float& s, uint32_t aw, uint32_t as) {
    if constexpr (BITS == 4) {
        uint2 v;
        asm volatile(
            "ds_read_b64 %0, %2\n\t"
            "ds_read_b32 %1, %3\n\t"
            "s_waitcnt lgkmcnt(0)"
            : "=&v"(v), "=&v"(s)
            : "v"(aw), "v"(as)
            : "memory");
        w[0] = v.x; w[1] = v.y;
    } else {
        uint4 v;
        asm volatile(
            "ds_read_b128 %0, %2\n\t"
            "ds_read_b32 %1, %3\n\t"
            "s_waitcnt lgkmcnt(0)"
            : "=&v"(v), "=&v"(s)
            : "v"(aw), "v"(as)
            : "memory");
        w[0] = v.x; w[1] = v.y; w[2] = v.z; w[3] = v.w;
    }
}

// W slot swizzle of local row r (0..31): 16-byte slots per row = K * BITS / 128.
template <int BITS>
__device__ __forceinline__ int w_swizzle(int r, bool odd_k256) {
    if constexpr (BITS == 4) return odd_k256 ? ((r >> 1) & 7) : (r & 15);
    else return r & 15;
}

template <int BITS, int SPW>
__global__ __launch_bounds__(512) void gemm_fwd_pipe_kernel(GemmArgs a, int tiles_i, int tiles_j, int per_xcd) {
    extern __shared__ __align__(16) float4 pipe_lds[];
    __shared__ float part[4 * 16 * 32];
    const int K = a.K;               // == 256 * SPW
    const int wspr = K * BITS / 128; // 16-byte W slots per row
    const bool odd = ((K >> 8) & 1) != 0;
    float4* xs = pipe_lds;                                    // [K/64 stages][16 rows][16 slots]
    float4* ws = pipe_lds + (K >> 6) * 256;                   // [32 rows][wspr slots]
    float* ss = reinterpret_cast<float*>(ws + 32 * wspr);     // [32 rows][groups]

    const int t = (blockIdx.x & 7) * per_xcd + (blockIdx.x >> 3);
    if (t >= tiles_i * tiles_j) return;
    const int ti = t / tiles_j, tj = t - ti * tiles_j;
    const int i0 = ti * 16, j0 = tj * 32;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int wk = wave & 3, wn = wave >> 2;
    const int r16 = lane & 15, q4 = lane >> 4;

    // Output element of this thread after the reduction, and its bias.
    const int e = threadIdx.x;
    const int oi = i0 + (e >> 5), oj = j0 + (e & 31);
    const float bb = a.has_bias ? a.bias[min(oj, a.cols - 1)] : 0.0f;
    __builtin_amdgcn_sched_barrier(0);

    // W codes of columns j0 .. j0+31, then their scales.
    const size_t row_bytes = size_t(K) * BITS / 8;
    const int winst = (32 * wspr) >> 6;
    for (int ii = wave; ii < winst; ii += 8) {
        const int L = ii * 64 + lane;
        const int row = L / wspr, pos = L - row * wspr;
        const uint8_t* src = static_cast<const uint8_t*>(a.B) + size_t(min(j0 + row, a.cols - 1)) * row_bytes +
                             (size_t(pos ^ w_swizzle<BITS>(row, odd)) << 4);
        __builtin_amdgcn_global_load_lds((global_cvoid*)src, (lds_void*)(ws + ii * 64), 16, 0, 0);
    }
    const int sslots = 8 * a.groups;   // 16-byte slots of the 32 x groups block
    for (int ii = wave; ii * 64 < sslots; ii += 8) {
        const int L = ii * 64 + lane;
        if (L < sslots) {
            const int f = 4 * L;
            const int row = f / a.groups, g = f - row * a.groups;
            const float* src = a.scale + size_t(min(j0 + row, a.cols - 1)) * a.groups + g;
            __builtin_amdgcn_global_load_lds((global_cvoid*)src, (lds_void*)(reinterpret_cast<float4*>(ss) + ii * 64),
                                             16, 0, 0);
        }
    }
    __builtin_amdgcn_sched_barrier(0);
    // X, stage by stage: this wave loads rows 8*wn .. 8*wn+7 of its stages.
#pragma unroll
    for (int u = 0; u < SPW; ++u) {
        const int st = wk + 4 * u;
#pragma unroll
        for (int cc = 0; cc < 2; ++cc) {
            const int c = 2 * wn + cc;
            const int row = 4 * c + (lane >> 4), p = lane & 15;
            const float* src = a.A + size_t(min(i0 + row, a.rows - 1)) * K + st * 64 + 4 * (p ^ row);
            __builtin_amdgcn_global_load_lds((global_cvoid*)src, (lds_void*)(xs + st * 256 + c * 64), 16, 0, 0);
        }
        __builtin_amdgcn_sched_barrier(0);
    }

    const int wrow = wn * 16 + r16;
    const int wsw = w_swizzle<BITS>(wrow, odd);
    uint32_t wc[SPW][BITS == 4 ? 2 : 4];
    float sc[SPW];
    f32x4 acc = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int u = 0; u < SPW; ++u) {
        // Everything this wave issued up to stage u has landed; the barrier
        // extends that to the other waves' loads of the same stages.
        if (u == SPW - 1) wait_own_loads_and_barrier<0>();
        else if (u == SPW - 2) wait_own_loads_and_barrier<2>();
        else if (u == SPW - 3) wait_own_loads_and_barrier<4>();
        else wait_own_loads_and_barrier<6>();
        if (u == 0) {
#pragma unroll
            for (int v = 0; v < SPW; ++v) {
                const int sv = wk + 4 * v;
                const int slot = BITS == 4 ? 2 * sv + (q4 >> 1) : 4 * sv + q4;
                const uint8_t* wp = reinterpret_cast<const uint8_t*>(ws + wrow * wspr + (slot ^ wsw)) +
                                    (BITS == 4 ? 8 * (q4 & 1) : 0);
                lds_read_codes<BITS>(wc[v], sc[v], lds_off(wp),
                                     lds_off(ss + wrow * a.groups + (sv * 64 + 16 * q4) / a.G));
            }
        }
        const int st = wk + 4 * u;
        const float4* xrow = xs + st * 256 + r16 * 16;
        float4 xv[4];
        lds_read_x4(xv[0], xv[1], xv[2], xv[3], lds_off(xrow + ((4 * q4 + 0) ^ r16)), lds_off(xrow + ((4 * q4 + 1) ^ r16)),
                    lds_off(xrow + ((4 * q4 + 2) ^ r16)), lds_off(xrow + ((4 * q4 + 3) ^ r16)));
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            const float4 x = xv[c];
            float bv[4];
            if constexpr (BITS == 8) {
                const uint32_t w = wc[u][c];
#pragma unroll
                for (int s2 = 0; s2 < 4; ++s2) bv[s2] = float(int(__builtin_amdgcn_sbfe(int(w), 8 * s2, 8))) * sc[u];
            } else {
                const uint32_t w = wc[u][c >> 1] >> (16 * (c & 1));
#pragma unroll
                for (int s2 = 0; s2 < 4; ++s2) bv[s2] = float(int(__builtin_amdgcn_sbfe(int(w), 4 * s2, 4))) * sc[u];
            }
            acc = __builtin_amdgcn_mfma_f32_16x16x4f32(x.x, bv[0], acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_f32_16x16x4f32(x.y, bv[1], acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_f32_16x16x4f32(x.z, bv[2], acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_f32_16x16x4f32(x.w, bv[3], acc, 0, 0, 0);
        }
        // Keep the next stage's wait below this stage's products.
        __builtin_amdgcn_sched_barrier(0);
    }

    // acc: rows 4*q4 + r, column wn*16 + r16. Parts summed in order 0..3, then the bias.
#pragma unroll
    for (int r = 0; r < 4; ++r) part[(wk * 16 + 4 * q4 + r) * 32 + wn * 16 + r16] = acc[r];
    __syncthreads();
    if (oi < a.rows && oj < a.cols) {
        float v = part[e];
#pragma unroll
        for (int p2 = 1; p2 < 4; ++p2) v += part[p2 * 512 + e];
        if (a.has_bias) v += bb;
        a.out[size_t(oi) * a.cols + oj] = v;
    }
}

size_t fwd_pipe_lds_bytes(const GemmArgs& a, int bits) {
    return size_t(16) * a.K * 4 + size_t(32) * a.K * bits / 8 + size_t(32) * a.groups * 4;
}

// int4 / int8 codes, 256 <= K <= 1024 with K % 256 == 0, groups of a multiple
// of 16 (one scale per lane per stage) with K / G % 4 == 0 (whole 16-byte scale
// slots per row), and 16-byte aligned X, codes and scales.
bool fwd_pipe_ok(const GemmArgs& a, int bits, const void* X, const void* W, const float* S) {
    if (bits != 4 && bits != 8) return false;
    if (a.K % 256 != 0 || a.K > 1024 || a.rows == 0 || a.cols == 0) return false;
    if (a.G % 16 != 0 || a.groups % 4 != 0) return false;
    return dgm::aligned(X, 16) && dgm::aligned(W, 16) && dgm::aligned(S, 16);
}

template <int BITS, int SPW>
int launch_fwd_pipe_spw(dgm_gpu* g, const GemmArgs& a) {
    const size_t lds = fwd_pipe_lds_bytes(a, BITS);
    if (lds > 64 * 1024) {
        hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(gemm_fwd_pipe_kernel<BITS, SPW>),
                                           hipFuncAttributeMaxDynamicSharedMemorySize, int(lds));
        if (e != hipSuccess)
            return dgm::fail(g, DGM_ERR_HIP, "gemm_nt: cannot reserve %zu bytes of LDS: %s", lds, hipGetErrorString(e));
    }
    const int ti = int(dgm::ceil_div(a.rows, 16)), tj = int(dgm::ceil_div(a.cols, 32));
    const int per = int((int64_t(ti) * tj + 7) / 8);
    hipLaunchKernelGGL((gemm_fwd_pipe_kernel<BITS, SPW>), dim3(unsigned(per) * 8u), dim3(512), lds, g->stream, a, ti,
                       tj, per);
    return DGM_OK;
}

template <int BITS>
int launch_fwd_pipe(dgm_gpu* g, const GemmArgs& a) {
    switch (a.K / 256) {
        case 1: return launch_fwd_pipe_spw<BITS, 1>(g, a);
        case 2: return launch_fwd_pipe_spw<BITS, 2>(g, a);
        case 3: return launch_fwd_pipe_spw<BITS, 3>(g, a);
        default: return launch_fwd_pipe_spw<BITS, 4>(g, a);
    }
}

// K % 64 == 0 and K <= 1024 (the X block stays in LDS; 512 with fp32
// weights, which take 16 registers per stage), a group that is a
// multiple of 16 (one scale per lane per stage), 16-byte aligned rows.
bool fwd_lds_ok(const GemmArgs& a, int bits, const void* X, const void* W) {
    if (a.K % 64 != 0 || a.K == 0 || a.K > 1024 || a.rows == 0 || a.cols == 0) return false;
    if (!dgm::aligned(X, 16)) return false;
    if (bits == 32) return a.K <= 512 && dgm::aligned(W, 16);
    if (a.G % 16 != 0) return false;
    return dgm::aligned(W, bits == 8 ? 16 : 8);
}

template <int BITS>
void launch_fwd_lds(const GemmArgs& a, int num_cus, hipStream_t st) {
    // Largest contraction split that leaves each part at least one stage and
    // the grid at least ~1.5 workgroups per CU.
    const int nst = a.K / 64;
    const int64_t ti = dgm::ceil_div(a.rows, 16);
    const int64_t w4 = ti * dgm::ceil_div(a.cols, 16), w2 = ti * dgm::ceil_div(a.cols, 32);
    if (nst >= 4 && (w2 < int64_t(num_cus) * 3 / 2 || nst >= 8)) {
        if (nst % 4 == 0) launch_fwd_reg<BITS>(a, st);
        else launch_fwd_lds_ks<BITS, 4>(a, st);
    }
    else if (nst >= 2 && w2 < int64_t(num_cus) * 3)
        launch_fwd_lds_ks<BITS, 2>(a, st);
    else
        launch_fwd_lds_ks<BITS, 1>(a, st);
    (void)w4;
}

// ---- LDS-staged STE dX for short contractions (N <= 448, N % 64 == 0) ---------
// dX[m, k] = sum_n dY[m, n] * deq(W)[n, k]. A workgroup owns 16 rows x 64
// columns of dX; each of its 4 waves owns 16 columns over the whole
// contraction. The 16 x N block of dY goes to LDS as in the forward (direct
// loads, swizzled slots). The weight strip W[0:N, k0:k0+64] is read with
// 16-byte loads (consecutive lanes take consecutive rows n) and written
// TRANSPOSED to LDS, [k][n], so that a lane's 4 consecutive contraction
// indices are one LDS read: dequantized once per workgroup (code * scale, the
// reference's rounding) as floats, rows padded to N + 4; or, with CODED, as
// one offset-binary byte per code (code + 8, code + 128; rows padded to N + 12
// bytes: at most two lanes per bank) with the scales per 16-k quarter of the
// strip as [quarter][n], each code dequantized when its operand is read,
// (byte - offset) * scale, the same single rounding. CODED holds 13 KB of
// codes instead of 49 KB of floats at N = 192: the backward pair, whose dX
// tiles otherwise leave room for only two workgroups per CU, takes it (c2:
// 8.2-8.5 us against 8.6-8.8); alone, the dequantization in the MFMA loop
// costs more than it saves (6.5-6.7 us against 5.9-6.1).
// RT = 2 gives the workgroup 32 rows (two accumulator tiles per wave on the
// same weight operands): half the strip loads and conversions per row of dX.
// The pair takes it when the tiles still fill the CUs (c2: 7.7-7.9 us
// against 8.4-8.5 us; fewer tiles or a 64-wide contraction lose).
// Contraction order inside a 64-wide stage is the same permutation for both
// operands (lane q takes 16q .. 16q+15), and every dX element is the same
// chain for either RT.
// Body of one dX tile; `blk` is the workgroup's index within its own grid
// (dealt round-robin to the 8 XCDs), sm4 its LDS (dx_lds_bytes(CODED, N, RT)).
template <int BITS, bool CODED = false, int RT = 1>
__device__ __forceinline__ void dx_lds_tile(const GemmArgs& a, int tiles_i, int tiles_j, int per_xcd, int blk,
                                            float4* sm4) {
    static_assert(!CODED || BITS != 32, "codes only");
    static_assert(RT == 1 || RT == 2, "16 or 32 rows");
    const int t = (blk & 7) * per_xcd + (blk >> 3);
    if (t >= tiles_i * tiles_j) return;
    const int ti = t / tiles_j, tj = t - ti * tiles_j;
    const int i0 = ti * 16 * RT, k0 = tj * 64;
    const int N = a.N, K = a.K;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int r16 = lane & 15, q4 = lane >> 4;
    const int spr = N >> 2;
    float4* ys = sm4;                                          // [16 RT][spr], swizzled
    float* wt = reinterpret_cast<float*>(sm4 + 16 * RT * spr);  // fp32: [64][N + 4]
    const int wld = N + 4;
    uint8_t* wc = reinterpret_cast<uint8_t*>(sm4 + 16 * RT * spr);  // codes: [64][N + 12] bytes
    const int wldb = N + 12;
    float* sc = reinterpret_cast<float*>(wc + 64 * wldb);      // codes: scales [4 quarters][N]

    // -- weight strip: 16-byte units. 32 consecutive lanes take 32 consecutive
    // rows n of one part of the strip, the next 32 lanes the next part, so a
    // wave instruction reads whole 32-byte (int4) row segments and the
    // transposed LDS writes below stay conflict-free. Units past the strip are
    // not loaded (units is a multiple of 64: N % 64 == 0).
    constexpr int CPU = BITS == 4 ? 32 : (BITS == 8 ? 16 : 4);   // codes (or floats) per unit
    constexpr int UPR = 64 / CPU;                                // units per row of the strip
    constexpr int MAXU = (448 * UPR + kThreads - 1) / kThreads;
    const int units = N * UPR;
    uint4 wv[MAXU];
    float ws[MAXU];
#pragma unroll
    for (int u = 0; u < MAXU; ++u) {
        if (u * kThreads >= units) break;
        const int idx = int(threadIdx.x) + u * kThreads;
        if (idx >= units) continue;   // wave-uniform (units % 64 == 0)
        const int grp = idx >> 5;
        const int n = (grp / UPR) * 32 + (idx & 31), part = grp % UPR;
        const int kc = min(k0 + part * CPU, K - CPU);   // strip columns past K: clamped, never stored
        if constexpr (BITS == 32) {
            wv[u] = *reinterpret_cast<const uint4*>(static_cast<const float*>(a.B) + size_t(n) * K + kc);
        } else {
            const size_t off = BITS == 8 ? size_t(n) * K + kc : (size_t(n) * K + kc) >> 1;
            wv[u] = *reinterpret_cast<const uint4*>(static_cast<const uint8_t*>(a.B) + off);
            ws[u] = a.scale[size_t(n) * a.groups + kc / a.G];
        }
    }
    // -- dY block via direct-to-LDS loads (slot pos of row r holds global slot pos ^ (r & 15)).
    const int ninst = (16 * RT * spr) >> 6;
    uint8_t* yb = reinterpret_cast<uint8_t*>(ys);
    for (int ii = wave; ii < ninst; ii += 4) {
        const int L = ii * 64 + lane;
        const int row = L / spr, pos = L - row * spr;
        const int gr = min(i0 + row, a.rows - 1);
        const float* src = a.A + size_t(gr) * N + ((pos ^ (row & 15)) << 2);
        __builtin_amdgcn_global_load_lds((global_cvoid*)src, (lds_void*)(yb + ii * 1024), 16, 0, 0);
    }
    // -- dequantize and transpose the strip into LDS.
#pragma unroll
    for (int u = 0; u < MAXU; ++u) {
        const int idx = int(threadIdx.x) + u * kThreads;
        if (idx >= units) break;
        const int grp = idx >> 5;
        const int n = (grp / UPR) * 32 + (idx & 31), part = grp % UPR;
        const uint32_t w4[4] = {wv[u].x, wv[u].y, wv[u].z, wv[u].w};
        if constexpr (BITS == 32) {
            float* dst = wt + (part * CPU) * wld + n;
#pragma unroll
            for (int e = 0; e < 4; ++e) dst[e * wld] = __uint_as_float(w4[e]);
        } else if constexpr (!CODED) {
            float* dst = wt + (part * CPU) * wld + n;
#pragma unroll
            for (int e = 0; e < CPU; ++e)
                dst[e * wld] = float(int(BITS == 8 ? __builtin_amdgcn_sbfe(int(w4[e >> 2]), 8 * (e & 3), 8)
                                                   : __builtin_amdgcn_sbfe(int(w4[e >> 3]), 4 * (e & 7), 4))) *
                               ws[u];
        } else {
            // Offset binary: a two's-complement nibble (byte) XOR its top bit.
            uint8_t* dst = wc + (part * CPU) * wldb + n;
#pragma unroll
            for (int e = 0; e < CPU; ++e) {
                const uint32_t b = BITS == 8 ? (w4[e >> 2] >> (8 * (e & 3))) & 0xFFu : (w4[e >> 3] >> (4 * (e & 7))) & 0xFu;
                dst[e * wldb] = uint8_t(b ^ (BITS == 8 ? 0x80u : 0x8u));
            }
#pragma unroll
            for (int qq = 0; qq < CPU / 16; ++qq) sc[(part * (CPU / 16) + qq) * N + n] = ws[u];
        }
    }
    __syncthreads();

    f32x4 acc[RT];
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) acc[rt] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    const float4* yrow = ys + r16 * spr;
    const float* wrow = wt + (wave * 16 + r16) * wld + 16 * q4;
    const uint8_t* crow = wc + (wave * 16 + r16) * wldb + 16 * q4;   // this lane's k row
    const float* srow = sc + wave * N + 16 * q4;                      // its quarter's scales
    constexpr float OFF = BITS == 8 ? 128.0f : 8.0f;
    const int nst = N >> 6;
    for (int st = 0; st < nst; ++st) {
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            float4 wv4;
            if constexpr (!CODED) {
                wv4 = *reinterpret_cast<const float4*>(wrow + st * 64 + 4 * c);
            } else {
                const uint32_t cb = *reinterpret_cast<const uint32_t*>(crow + st * 64 + 4 * c);
                const float4 s4 = *reinterpret_cast<const float4*>(srow + st * 64 + 4 * c);
                // (code + OFF) - OFF is exact; one rounding in the product.
                wv4.x = (float(cb & 0xFFu) - OFF) * s4.x;
                wv4.y = (float((cb >> 8) & 0xFFu) - OFF) * s4.y;
                wv4.z = (float((cb >> 16) & 0xFFu) - OFF) * s4.z;
                wv4.w = (float(cb >> 24) - OFF) * s4.w;
            }
#pragma unroll
            for (int rt = 0; rt < RT; ++rt) {
                const float4 yv = yrow[rt * 16 * spr + ((st * 16 + 4 * q4 + c) ^ r16)];
                acc[rt] = __builtin_amdgcn_mfma_f32_16x16x4f32(yv.x, wv4.x, acc[rt], 0, 0, 0);
                acc[rt] = __builtin_amdgcn_mfma_f32_16x16x4f32(yv.y, wv4.y, acc[rt], 0, 0, 0);
                acc[rt] = __builtin_amdgcn_mfma_f32_16x16x4f32(yv.z, wv4.z, acc[rt], 0, 0, 0);
                acc[rt] = __builtin_amdgcn_mfma_f32_16x16x4f32(yv.w, wv4.w, acc[rt], 0, 0, 0);
            }
        }
    }
    const int k = k0 + wave * 16 + r16;
    if (k < K) {
        if (a.sg_gate) {
            // All rows' gate and up values are loaded before the first store,
            // so no store waits on a later row's loads.
            float gv[RT][4], uv[RT][4];
#pragma unroll
            for (int rt = 0; rt < RT; ++rt)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const size_t e = size_t(min(i0 + 16 * rt + 4 * q4 + r, a.rows - 1)) * K + k;
                    gv[rt][r] = a.sg_gate[e];
                    uv[rt][r] = a.sg_up[e];
                }
#pragma unroll
            for (int rt = 0; rt < RT; ++rt)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int i = i0 + 16 * rt + 4 * q4 + r;
                    if (i < a.rows) {
                        float* o = a.out + size_t(i) * 2 * K + k;
                        dgm::swiglu_bwd_value(gv[rt][r], uv[rt][r], acc[rt][r], o[0], o[K]);
                    }
                }
        } else {
#pragma unroll
            for (int rt = 0; rt < RT; ++rt)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int i = i0 + 16 * rt + 4 * q4 + r;
                    if (i < a.rows) a.out[size_t(i) * K + k] = acc[rt][r];
                }
        }
    }
}

template <int BITS>
__global__ __launch_bounds__(kThreads) void gemm_dx_lds_kernel(GemmArgs a, int tiles_i, int tiles_j, int per_xcd) {
    extern __shared__ __align__(16) float4 sm4[];
    dx_lds_tile<BITS>(a, tiles_i, tiles_j, per_xcd, int(blockIdx.x), sm4);
}

size_t dx_lds_bytes(bool coded, int N, int rt = 1) {
    const size_t strip = coded ? size_t(64) * (N + 12) + size_t(4) * N * 4 : size_t(64) * (N + 4) * 4;
    return size_t(16) * rt * N * 4 + strip;
}

// N % 64 == 0 and N <= 448 (dY block and the transposed strip stay in LDS),
// K a multiple of the 16-byte unit, a group that holds a whole unit, aligned rows.
bool dx_lds_ok(const GemmArgs& a, int bits, const void* dY, const void* W) {
    if (a.N % 64 != 0 || a.N == 0 || a.N > 448 || a.rows == 0 || a.K == 0) return false;
    if (!dgm::aligned(dY, 16) || !dgm::aligned(W, 16)) return false;
    const int cpu = bits == 4 ? 32 : (bits == 8 ? 16 : 4);
    if (a.K % cpu != 0) return false;
    return bits == 32 || a.G % cpu == 0;
}

template <int BITS>
int launch_dx_lds(dgm_gpu* g, const GemmArgs& a) {
    const size_t lds = dx_lds_bytes(false, a.N);
    if (lds > 64 * 1024) {
        hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(gemm_dx_lds_kernel<BITS>),
                                           hipFuncAttributeMaxDynamicSharedMemorySize, int(lds));
        if (e != hipSuccess)
            return dgm::fail(g, DGM_ERR_HIP, "gemm_dx: cannot reserve %zu bytes of LDS: %s", lds, hipGetErrorString(e));
    }
    const int ti = int(dgm::ceil_div(a.rows, 16)), tj = int(dgm::ceil_div(a.K, 64));
    const int64_t nt = int64_t(ti) * tj;
    const int per = int((nt + 7) / 8);
    hipLaunchKernelGGL(gemm_dx_lds_kernel<BITS>, dim3(unsigned(per) * 8u), dim3(kThreads), lds, g->stream, a, ti, tj,
                       per);
    return DGM_OK;
}

// ---- dW with 2 or 4 columns per lane (M % 64 == 0, N % NP == 0) ------------------
// The tile is dgm_dw::dw_tile (dw_tile.hpp): 16 NP rows (n) x 16 columns (k),
// four waves splitting M, CH 16-row chunks of loads per round. The 32 x 16
// tile (NP = 2) takes two chunks per round (kPairCH): fewer registers, more
// workgroups per CU (c2 pair 7.5-7.6 us against 7.8-7.9 with eight; the DiT
// training step 324 us against 331; dW alone 2-7% faster at the 32-row
// shapes; one chunk and four measured no better). The 64 x 16 tile (NP = 4,
// CH = 4, 110 VGPRs) runs dW alone where launch_dw_pair finds it pays (c2 /
// c1: 5.4 us against 6.7 us). The deep-dX pair keeps eight chunks (two
// measured 3% slower at the c1 shape).
constexpr int DWP_CH = 8;                    // 16-row chunks per wave and round beside the deep dX tiles
constexpr int kPairCH = dgm_dw::kPairCH;     // the same for the 32 x 16 tiles elsewhere

// Body of one dW tile of a 256-thread workgroup; `blk` as in dx_lds_tile,
// part: NP x 4 KB of LDS.
template <int NP = 2, int CH = DWP_CH>
__device__ __forceinline__ void dw_pair_tile(const GemmArgs& a, int tiles_n, int tiles_k, int per_xcd, int blk,
                                             float (*part)[NP][16][16]) {
    const int t = (blk & 7) * per_xcd + (blk >> 3);
    if (t >= tiles_n * tiles_k) return;   // the whole workgroup: no barrier is skipped by part of it
    const dgm_dw::DwTileArgs d{a.A, static_cast<const float*>(a.B), a.out, a.M, a.N, a.K, a.accumulate};
    dgm_dw::dw_tile<NP, CH>(d, true, t, tiles_n, int(threadIdx.x >> 6), int(threadIdx.x), part);
}

template <int NP, int CH>
__global__ __launch_bounds__(kThreads) void gemm_dw_pair_kernel(GemmArgs a, int tiles_n, int tiles_k, int per_xcd) {
    __shared__ float part[4][NP][16][16];
    dw_pair_tile<NP, CH>(a, tiles_n, tiles_k, per_xcd, int(blockIdx.x), part);
}

// ---- the STE backward pair in one launch ------------------------------------------
// Workgroups [0, 8*per_x) compute dX tiles (dx_lds_tile), the rest dW tiles
// (dw_pair_tile): the two GEMMs share no output and only read dY, so they run
// side by side instead of back to back. Each tile's elements are computed as
// by its own kernel (dX tiles of 16 RT rows).
template <int BITS, int RT>
__global__ __launch_bounds__(kThreads) void gemm_bwd_pair_kernel(GemmArgs ax, int ti, int tj, int per_x, GemmArgs aw,
                                                                 int tn, int tk, int per_w) {
    extern __shared__ __align__(16) float4 sm4[];
    const int nx = 8 * per_x;
    if (int(blockIdx.x) < nx) {
        dx_lds_tile<BITS, BITS != 32, RT>(ax, ti, tj, per_x, int(blockIdx.x), sm4);
    } else {
        dw_pair_tile<2, kPairCH>(aw, tn, tk, per_w, int(blockIdx.x) - nx, reinterpret_cast<float (*)[2][16][16]>(sm4));
    }
}

// The same pairing for contractions too long for the LDS dX kernel: 16 x 32
// deep-prefetch dX tiles (gemm_deep_kernel<MODE_DX, BITS, 16, 32, 8>) beside
// the paired-column dW tiles (16 x 32 measured ~2% faster than 16 x 16 in the
// DiT backward).
constexpr int kDeepPairTN = 32, kDeepPairPF = 8;   // dX tile width and prefetch depth of the pair

template <int BITS>
__global__ __launch_bounds__(kThreads) void gemm_bwd_deep_pair_kernel(GemmArgs ax, int ti, int tj, int per_x,
                                                                      GemmArgs aw, int tn, int tk, int per_w) {
    extern __shared__ __align__(16) float4 sm4[];
    const int nx = 8 * per_x;
    if (int(blockIdx.x) < nx) {
        deep_tile<MODE_DX, BITS, 16, kDeepPairTN, kDeepPairPF>(ax, ti, tj, per_x, int(blockIdx.x),
                                                                reinterpret_cast<float (*)[16 * kDeepPairTN]>(sm4));
    } else {
        dw_pair_tile(aw, tn, tk, per_w, int(blockIdx.x) - nx, reinterpret_cast<float (*)[2][16][16]>(sm4));
    }
}

bool dw_pair_ok(const GemmArgs& a, const void* dY) {
    return a.M > 0 && a.M % 64 == 0 && a.N >= 2 && a.N % 2 == 0 && a.K > 0 && dgm::aligned(dY, 8);
}

// 64-row tiles (four dY columns per lane) do a 32-row tile's work in ~1.65x
// its time; they pay when they need fewer rounds of workgroups over the CUs
// by more than that factor (measured at M = 512..2048, N x K from 192 x 192 to
// 4096 x 1024: e.g. 192 x 768 5.75 against 6.9 us, 192 x 192 6.3 against 4.8).
void launch_dw_pair(const GemmArgs& a, int num_cus, hipStream_t st) {
    const int64_t nc = num_cus > 0 ? num_cus : 1, tk64 = dgm::ceil_div(a.K, 16);
    const int64_t r2 = (dgm::ceil_div(a.N, 32) * tk64 + nc - 1) / nc, r4 = (dgm::ceil_div(a.N, 64) * tk64 + nc - 1) / nc;
    const bool four = a.N % 4 == 0 && dgm::aligned(a.A, 16) && 33 * r4 < 20 * r2;
    const int tn = int(dgm::ceil_div(a.N, four ? 64 : 32)), tk = int(dgm::ceil_div(a.K, 16));
    const int64_t nt = int64_t(tn) * tk;
    const int per = int((nt + 7) / 8);
    if (four)
        hipLaunchKernelGGL((gemm_dw_pair_kernel<4, 4>), dim3(unsigned(per) * 8u), dim3(kThreads), 0, st, a, tn, tk, per);
    else
        hipLaunchKernelGGL((gemm_dw_pair_kernel<2, kPairCH>), dim3(unsigned(per) * 8u), dim3(kThreads), 0, st, a, tn,
                           tk, per);
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


// ---- dX on bf16 MFMA with the group scale folded into dY ---------------------------
// dX[m,k] = sum_n dY[m,n] * code[n,k] * S[n, k/G]. For the columns of one
// 32-wide block (inside one group g), A[m,n] = dY[m,n] * S[n,g] (one fp32
// rounding, as the reference's code * scale) split into three bf16 pieces
// hi + mid + lo that sum to it exactly, and B = the codes (integers of at most
// 8 bits, exact in bf16): three v_mfma_f32_16x16x32_bf16 per 32-n step, the
// products exact, the sum in fp32. The codes and scales come transposed
// (codesT [K][N] int8, scalesT [K/G][N]), made once per weight by
// wt_prep_kernel, so a lane's 8 consecutive n are one 8-byte load.
// A workgroup owns 16 rows x 32 columns; its 4 waves take interleaved 32-n
// steps and their partial tiles are added in wave order through LDS.
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ uint32_t pk_bf16(float a, float b) {
    const f32x2 v = {a, b};
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2));
}

// Three bf16 pieces of 8 values: v = hi + mid + lo exactly (truncation).
__device__ __forceinline__ void pieces8(const float (&v)[8], bf16x8& hi, bf16x8& mi, bf16x8& lo) {
    u32x4 h, m, l;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        float x0 = v[2 * i], x1 = v[2 * i + 1];
        const float h0 = __uint_as_float(__float_as_uint(x0) & 0xFFFF0000u);
        const float h1 = __uint_as_float(__float_as_uint(x1) & 0xFFFF0000u);
        x0 = x0 - h0;
        x1 = x1 - h1;
        const float m0 = __uint_as_float(__float_as_uint(x0) & 0xFFFF0000u);
        const float m1 = __uint_as_float(__float_as_uint(x1) & 0xFFFF0000u);
        h[i] = pk_bf16(h0, h1);
        m[i] = pk_bf16(m0, m1);
        l[i] = pk_bf16(x0 - m0, x1 - m1);
    }
    hi = __builtin_bit_cast(bf16x8, h);
    mi = __builtin_bit_cast(bf16x8, m);
    lo = __builtin_bit_cast(bf16x8, l);
}

__device__ __forceinline__ bf16x8 i8x8_bf16(uint2 w) {
    u32x4 r;
    r.x = pk_bf16(float(int8_t(w.x)), float(int8_t(w.x >> 8)));
    r.y = pk_bf16(float(int8_t(w.x >> 16)), float(int8_t(w.x >> 24)));
    r.z = pk_bf16(float(int8_t(w.y)), float(int8_t(w.y >> 8)));
    r.w = pk_bf16(float(int8_t(w.y >> 16)), float(int8_t(w.y >> 24)));
    return __builtin_bit_cast(bf16x8, r);
}

struct DxFoldArgs {
    const float* dY;          // [M, N]
    const int8_t* codesT;     // [K][N]
    const float* scalesT;     // [K/G][N]
    float* out;               // [M, K], or [M, 2K] rows [dgate | dup] with the SwiGLU backward
    const float *sg_gate, *sg_up;   // [M, K] or null
    int M, N, K, G;
};

constexpr int kFoldSteps = 2;   // 32-n steps whose loads are in flight together per wave

__device__ __forceinline__ void dx_fold_tile(const DxFoldArgs& a, int tiles_m, int tiles_k, int per_xcd, int blk,
                                             float (*part)[2][16][16]) {
#pragma clang fp contract(off)
    const int t = (blk & 7) * per_xcd + (blk >> 3);
    if (t >= tiles_m * tiles_k) return;
    const int tk = t / tiles_m, tm = t - tk * tiles_m;   // consecutive tiles share a column block
    const int m0 = tm * 16, k0 = tk * 32, g = k0 / a.G;
    const int N = a.N, K = a.K;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int r16 = lane & 15, q4 = lane >> 4;
    const float* yrow = a.dY + size_t(min(m0 + r16, a.M - 1)) * N + 8 * q4;
    const float* srow = a.scalesT + size_t(g) * N + 8 * q4;
    const int8_t* c0 = a.codesT + size_t(k0 + r16) * N + 8 * q4;
    const int8_t* c1 = c0 + size_t(16) * N;
    f32x4 acc0 = f32x4{0.0f, 0.0f, 0.0f, 0.0f}, acc1 = acc0;
    const int steps = N / 32;
    for (int s0 = wave; s0 < steps; s0 += 4 * kFoldSteps) {
        float4 yv[kFoldSteps][2], sv[kFoldSteps][2];
        uint2 w0[kFoldSteps], w1[kFoldSteps];
#pragma unroll
        for (int u = 0; u < kFoldSteps; ++u) {
            const int s = min(s0 + 4 * u, steps - 1);   // past the end: re-read, not computed
            const int n = 32 * s;
            yv[u][0] = *reinterpret_cast<const float4*>(yrow + n);
            yv[u][1] = *reinterpret_cast<const float4*>(yrow + n + 4);
            sv[u][0] = *reinterpret_cast<const float4*>(srow + n);
            sv[u][1] = *reinterpret_cast<const float4*>(srow + n + 4);
            w0[u] = *reinterpret_cast<const uint2*>(c0 + n);
            w1[u] = *reinterpret_cast<const uint2*>(c1 + n);
        }
#pragma unroll
        for (int u = 0; u < kFoldSteps; ++u) {
            if (s0 + 4 * u >= steps) break;
            const float v[8] = {yv[u][0].x * sv[u][0].x, yv[u][0].y * sv[u][0].y, yv[u][0].z * sv[u][0].z,
                                yv[u][0].w * sv[u][0].w, yv[u][1].x * sv[u][1].x, yv[u][1].y * sv[u][1].y,
                                yv[u][1].z * sv[u][1].z, yv[u][1].w * sv[u][1].w};
            bf16x8 hi, mi, lo;
            pieces8(v, hi, mi, lo);
            const bf16x8 b0 = i8x8_bf16(w0[u]), b1 = i8x8_bf16(w1[u]);
            acc0 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(lo, b0, acc0, 0, 0, 0);
            acc1 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(lo, b1, acc1, 0, 0, 0);
            acc0 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(mi, b0, acc0, 0, 0, 0);
            acc1 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(mi, b1, acc1, 0, 0, 0);
            acc0 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(hi, b0, acc0, 0, 0, 0);
            acc1 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(hi, b1, acc1, 0, 0, 0);
        }
    }
    // acc_t[r]: row m0 + 4 q4 + r, column k0 + 16 t + r16.
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        part[wave][0][4 * q4 + r][r16] = acc0[r];
        part[wave][1][4 * q4 + r][r16] = acc1[r];
    }
    __syncthreads();
    for (int e = threadIdx.x; e < 16 * 32; e += kThreads) {
        const int il = e >> 5, j = e & 31, tt = j >> 4, jj = j & 15;
        const int i = m0 + il, k = k0 + j;
        if (i >= a.M) continue;
        float v = part[0][tt][il][jj];
        v += part[1][tt][il][jj];
        v += part[2][tt][il][jj];
        v += part[3][tt][il][jj];
        if (a.sg_gate) {
            const size_t ei = size_t(i) * K + k;
            float* o = a.out + size_t(i) * 2 * K + k;
            dgm::swiglu_bwd_value_hw(a.sg_gate[ei], a.sg_up[ei], v, o[0], o[K]);
        } else {
            a.out[size_t(i) * K + k] = v;
        }
    }
}

// dX tiles (dx_fold_tile) beside the paired-column dW tiles (dw_pair_tile).
__global__ __launch_bounds__(kThreads) void gemm_bwd_fold_pair_kernel(DxFoldArgs ax, int tm, int tk, int per_x,
                                                                      GemmArgs aw, int tn, int tkw, int per_w) {
    __shared__ float part[4][2][16][16];
    const int nx = 8 * per_x;
    if (int(blockIdx.x) < nx) dx_fold_tile(ax, tm, tk, per_x, int(blockIdx.x), part);
    else dw_pair_tile<2, kPairCH>(aw, tn, tkw, per_w, int(blockIdx.x) - nx, part);
}

// codesT[k][n] = code[n][k] (int8, also for int4 codes) and scalesT[g][n] =
// S[n][g] of one linear, through 64 x 64 LDS tiles. Linears li = 0 .. nlin-1
// take consecutive runs of workgroups.
struct WtPrepArgs {
    const void* W[4];
    const float* S[4];
    int8_t* codesT[4];
    float* scalesT[4];
    int N[4], K[4], G[4];
    int first[5];   // first workgroup of each linear
    int nlin;
};

template <int BITS>
__global__ __launch_bounds__(kThreads) void wt_prep_kernel(WtPrepArgs a) {
    __shared__ __align__(16) int8_t tile[64][64 + 16];
    int li = 0;
    while (li + 1 < a.nlin && int(blockIdx.x) >= a.first[li + 1]) ++li;
    const int N = a.N[li], K = a.K[li], G = a.G[li];
    const int tiles_n = (N + 63) / 64;
    const int t = int(blockIdx.x) - a.first[li];
    const int n0 = (t % tiles_n) * 64, k0 = (t / tiles_n) * 64;
    const int tid = threadIdx.x;
    const int r = tid >> 2, c = (tid & 3) * 16;   // row r, codes c .. c+15 of the tile
    // 64 rows x 64 codes: one 16-byte (int8) / 8-byte (int4) load per thread
    // (K % 32 == 0: a run of 16 lies wholly inside or outside the matrix).
    {
        const int n = n0 + r, k = k0 + c;
        uint32_t wv[4] = {0u, 0u, 0u, 0u};
        if (n < N && k < K) {
            if constexpr (BITS == 8) {
                const uint4 q = *reinterpret_cast<const uint4*>(static_cast<const int8_t*>(a.W[li]) + size_t(n) * K + k);
                wv[0] = q.x; wv[1] = q.y; wv[2] = q.z; wv[3] = q.w;
            } else {
                const uint2 q =
                    *reinterpret_cast<const uint2*>(static_cast<const uint8_t*>(a.W[li]) + ((size_t(n) * K + k) >> 1));
#pragma unroll
                for (int h = 0; h < 2; ++h) {   // 8 nibbles (low first) -> 8 sign-extended bytes
                    const uint32_t x = h ? q.y : q.x;
#pragma unroll
                    for (int j = 0; j < 8; ++j) {
                        const uint32_t b = uint32_t(int32_t(x << (28 - 4 * j)) >> 28) & 0xFFu;
                        wv[2 * h + j / 4] |= b << (8 * (j % 4));
                    }
                }
            }
        }
#pragma unroll
        for (int i = 0; i < 16; ++i) tile[c + i][r] = int8_t(wv[i / 4] >> (8 * (i % 4)));
    }
    __syncthreads();
    {
        const int k = k0 + r, n = n0 + c;   // row k of the transpose, n .. n+15 (N % 32 == 0)
        if (k < K && n < N)
            *reinterpret_cast<uint4*>(a.codesT[li] + size_t(k) * N + n) = *reinterpret_cast<const uint4*>(&tile[r][c]);
    }
    // scales: the workgroups of the first column block transpose their rows.
    if (k0 == 0) {
        const int groups = K / G;
        for (int e = tid; e < 64 * groups; e += kThreads) {
            const int gg = e / 64, n = n0 + e % 64;
            if (n < N) a.scalesT[li][size_t(gg) * N + n] = a.S[li][size_t(n) * groups + gg];
        }
    }
}

}  // namespace

namespace dgm {

bool skinny_ok(int bits, const void* W, const float* X, const dgm_GemmP* p);
bool skinny_fused_ok(dgm_gpu* g, int bits, const void* W, const float* X, const dgm_GemmP* p);
bool decode_ok(int bits, const void* W, const float* X, const float* S, const dgm_GemmP* p);
int decode_fwd(dgm_gpu* g, int bits, const void* W, const float* scale, const float* X, const float* bias, float* Y,
               const dgm_GemmP* p);
int skinny_fwd(dgm_gpu* g, int bits, const void* W, const float* scale, const float* X,
               const float* bias, float* Y, const dgm_GemmP* p);
bool bf16_ok(int bits, const void* W, const float* X, const float* S, const dgm_GemmP* p);
bool stream_ok(dgm_gpu* g, int bits, const void* W, const float* X, const float* S, const dgm_GemmP* p);
bool slab_ok(dgm_gpu* g, int bits, const void* W, const float* X, const float* S, const dgm_GemmP* p);
int slab_fwd(dgm_gpu* g, int bits, const void* W, const float* scale, const float* X, const float* bias, float* Y,
             const dgm_GemmP* p);
int stream_fwd(dgm_gpu* g, int bits, const void* W, const float* scale, const float* X, const float* bias, float* Y,
               const dgm_GemmP* p);
int bf16_fwd(dgm_gpu* g, int bits, const void* W, const float* scale, const float* X,
             const float* bias, float* Y, const dgm_GemmP* p);

// Entry used by the dispatcher in gemm_entry.hip; declared there.
int gemm_f32_fwd(dgm_gpu* g, int bits, const void* W, const float* scale, const float* X,
                 const float* bias, float* Y, const dgm_GemmP* p) {
    // Decode-shaped quantized forwards stream W once. GEMV-like calls (a few
    // rows) take the int8-MFMA kernel, whose weight unpack is three bit
    // operations per 8 weights and whose activation pieces fill spare MFMA
    // rows; up to 16 rows (8 in the reduced mode) split K over workgroups on
    // the same arithmetic when the weights are large (gemm_slab.hip); more
    // rows take f16 MFMA over exact f16 activation pieces (gemm_decode.hip),
    // or the int8-MFMA kernel outside those domains.
    if (stream_ok(g, bits, W, X, scale, p)) return stream_fwd(g, bits, W, scale, X, bias, Y, p);
    if (slab_ok(g, bits, W, X, scale, p)) return slab_fwd(g, bits, W, scale, X, bias, Y, p);
    if (skinny_fused_ok(g, bits, W, X, p)) return skinny_fwd(g, bits, W, scale, X, bias, Y, p);
    if (decode_ok(bits, W, X, scale, p)) return decode_fwd(g, bits, W, scale, X, bias, Y, p);
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
    // The pipelined 16 x 32 kernel where the 4-way contraction split applies:
    // at least 1.5 tiles per CU would otherwise be too few, or K >= 512.
    if (fwd_pipe_ok(a, bits, X, W, scale)) {
        const int64_t w2 = int64_t(dgm::ceil_div(a.rows, 16)) * dgm::ceil_div(a.cols, 32);
        if (w2 < int64_t(g->num_cus) * 3 / 2 || a.K >= 512)
            return bits == 8 ? launch_fwd_pipe<8>(g, a) : launch_fwd_pipe<4>(g, a);
    }
    if (fwd_lds_ok(a, bits, X, W)) {
        if (bits == 32) launch_fwd_lds<32>(a, g->num_cus, g->stream);
        else if (bits == 8) launch_fwd_lds<8>(a, g->num_cus, g->stream);
        else launch_fwd_lds<4>(a, g->num_cus, g->stream);
        return DGM_OK;
    }
    if (deep_ok<MODE_FWD>(a, bits, vec)) {
        if (bits == 32) launch_deep<MODE_FWD, 32>(a, g->num_cus, g->stream);
        else if (bits == 8) launch_deep<MODE_FWD, 8>(a, g->num_cus, g->stream);
        else launch_deep<MODE_FWD, 4>(a, g->num_cus, g->stream);
        return DGM_OK;
    }
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
    if (dx_lds_ok(a, bits, dY, W)) {
        if (bits == 32) return launch_dx_lds<32>(g, a);
        if (bits == 8) return launch_dx_lds<8>(g, a);
        return launch_dx_lds<4>(g, a);
    }
    if (deep_ok<MODE_DX>(a, bits, vec)) {
        if (bits == 32) launch_deep<MODE_DX, 32>(a, g->num_cus, g->stream);
        else if (bits == 8) launch_deep<MODE_DX, 8>(a, g->num_cus, g->stream);
        else launch_deep<MODE_DX, 4>(a, g->num_cus, g->stream);
        return DGM_OK;
    }
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
    if (dw_pair_ok(a, dY)) {
        launch_dw_pair(a, g->num_cus, g->stream);
        return DGM_OK;
    }
    if (deep_ok<MODE_DW>(a, 32, false)) launch_deep<MODE_DW, 32>(a, g->num_cus, g->stream);
    else launch_gemm<MODE_DW, 32>(a, false, g->num_cus, g->stream);
    return DGM_OK;
}

// dX and dW of one linear as a single launch (gemm_bwd_pair_kernel) when both
// shapes take the LDS dX kernel and the paired-column dW kernel; *fused tells
// the caller whether it ran (else it runs gemm_f32_dx and gemm_f32_dw). With
// sg_gate / sg_up, dX leaves as the SwiGLU backward [dgate | dup] rows.
int gemm_f32_bwd_pair(dgm_gpu* g, int bits, const void* W, const float* scale, const float* dY, const float* X,
                      float* dX, float* dW, const dgm_GemmP* p, bool accumulate, bool* fused, const float* sg_gate,
                      const float* sg_up) {
    *fused = false;
    GemmArgs ax{};
    ax.A = dY; ax.B = W; ax.scale = scale; ax.out = dX;
    ax.sg_gate = sg_gate; ax.sg_up = sg_up;
    ax.M = p->M; ax.N = p->N; ax.K = p->K;
    ax.rows = p->M; ax.cols = p->K; ax.red = p->N;
    ax.G = bits == 32 ? 1 : int(p->qGroup);
    ax.groups = bits == 32 ? 0 : int(p->K / p->qGroup);
    GemmArgs aw{};
    aw.A = dY; aw.B = X; aw.out = dW;
    aw.M = p->M; aw.N = p->N; aw.K = p->K;
    aw.rows = p->N; aw.cols = p->K; aw.red = p->M;
    aw.G = 1; aw.groups = 0;
    aw.accumulate = accumulate;
    if (!dw_pair_ok(aw, dY)) return DGM_OK;
    if (!dx_lds_ok(ax, bits, dY, W)) {
        // Deep dX tiles beside the dW tiles, where gemm_f32_dx would pick the
        // 16 x 16 deep kernel (no SwiGLU epilogue there).
        const bool vec = (p->N % 4) == 0 && aligned(dY, 16);
        const int64_t t16x32 = int64_t(dgm::ceil_div(ax.rows, 16)) * dgm::ceil_div(ax.cols, 32);
        if (sg_gate || !deep_ok<MODE_DX>(ax, bits, vec) || t16x32 >= 2 * g->num_cus) return DGM_OK;
        const int ti = int(dgm::ceil_div(ax.rows, 16)), tj = int(dgm::ceil_div(ax.cols, kDeepPairTN));
        const int per_x = int((int64_t(ti) * tj + 7) / 8);
        const int tn = int(dgm::ceil_div(aw.N, 32)), tk = int(dgm::ceil_div(aw.K, 16));
        const int per_w = int((int64_t(tn) * tk + 7) / 8);
        const dim3 grid(unsigned(per_x + per_w) * 8u);
        const size_t lds = 8 * 1024;   // dW tiles: 8 KB; dX tiles: 4 x 16 x kDeepPairTN floats
        if (bits == 32)
            hipLaunchKernelGGL(gemm_bwd_deep_pair_kernel<32>, grid, dim3(kThreads), lds, g->stream, ax, ti, tj, per_x,
                               aw, tn, tk, per_w);
        else if (bits == 8)
            hipLaunchKernelGGL(gemm_bwd_deep_pair_kernel<8>, grid, dim3(kThreads), lds, g->stream, ax, ti, tj, per_x,
                               aw, tn, tk, per_w);
        else
            hipLaunchKernelGGL(gemm_bwd_deep_pair_kernel<4>, grid, dim3(kThreads), lds, g->stream, ax, ti, tj, per_x,
                               aw, tn, tk, per_w);
        *fused = true;
        return DGM_OK;
    }
    // 32-row dX tiles (coded strips) when N >= 128 and they still give at
    // least half as many workgroups as CUs; else 16 rows.
    const int rt = (bits != 32 && ax.N >= 128 &&
                    int64_t(dgm::ceil_div(ax.rows, 32)) * dgm::ceil_div(ax.K, 64) * 2 >= g->num_cus)
                       ? 2
                       : 1;
    const size_t lds = dx_lds_bytes(bits != 32, ax.N, rt);   // >= the 8 KB the dW tiles use (N >= 64)
    const void* kern =
        bits == 32 ? reinterpret_cast<const void*>(gemm_bwd_pair_kernel<32, 1>)
        : bits == 8 ? (rt == 2 ? reinterpret_cast<const void*>(gemm_bwd_pair_kernel<8, 2>)
                               : reinterpret_cast<const void*>(gemm_bwd_pair_kernel<8, 1>))
                    : (rt == 2 ? reinterpret_cast<const void*>(gemm_bwd_pair_kernel<4, 2>)
                               : reinterpret_cast<const void*>(gemm_bwd_pair_kernel<4, 1>));
    if (lds > 64 * 1024) {
        hipError_t e = hipFuncSetAttribute(kern, hipFuncAttributeMaxDynamicSharedMemorySize, int(lds));
        if (e != hipSuccess)
            return dgm::fail(g, DGM_ERR_HIP, "gemm_bwd: cannot reserve %zu bytes of LDS: %s", lds,
                             hipGetErrorString(e));
    }
    const int ti = int(dgm::ceil_div(ax.rows, 16 * rt)), tj = int(dgm::ceil_div(ax.K, 64));
    const int per_x = int((int64_t(ti) * tj + 7) / 8);
    const int tn = int(dgm::ceil_div(aw.N, 32)), tk = int(dgm::ceil_div(aw.K, 16));
    const int per_w = int((int64_t(tn) * tk + 7) / 8);
    const dim3 grid(unsigned(per_x + per_w) * 8u);
#define DGM_PAIR_LAUNCH(B, R) \
    hipLaunchKernelGGL((gemm_bwd_pair_kernel<B, R>), grid, dim3(kThreads), lds, g->stream, ax, ti, tj, per_x, aw, tn, tk, per_w)
    if (bits == 32) DGM_PAIR_LAUNCH(32, 1);
    else if (bits == 8 && rt == 2) DGM_PAIR_LAUNCH(8, 2);
    else if (bits == 8) DGM_PAIR_LAUNCH(8, 1);
    else if (rt == 2) DGM_PAIR_LAUNCH(4, 2);
    else DGM_PAIR_LAUNCH(4, 1);
#undef DGM_PAIR_LAUNCH
    *fused = true;
    return DGM_OK;
}

// ---- dX on bf16 MFMA beside the fp32 dW tiles (the DiT backward's linears) ---------
int wt_prep(dgm_gpu* g, int bits, int nlin, const void* const* W, const float* const* S, const int* N, const int* K,
            int G, int8_t* const* codesT, float* const* scalesT) {
    if (nlin <= 0 || nlin > 4) return fail(g, DGM_ERR_ARG, "wt_prep: %d linears", nlin);
    for (int i = 0; i < nlin; ++i)
        if (N[i] % 32 != 0 || K[i] % 32 != 0 || !aligned(W[i], bits == 8 ? 16 : 8) || !aligned(codesT[i], 16))
            return fail(g, DGM_ERR_UNSUPPORTED, "wt_prep: sizes or alignment");
    WtPrepArgs a{};
    a.nlin = nlin;
    int blocks = 0;
    for (int i = 0; i < nlin; ++i) {
        a.W[i] = W[i]; a.S[i] = S[i]; a.codesT[i] = codesT[i]; a.scalesT[i] = scalesT[i];
        a.N[i] = N[i]; a.K[i] = K[i]; a.G[i] = G;
        a.first[i] = blocks;
        blocks += int(ceil_div(N[i], 64) * ceil_div(K[i], 64));
    }
    a.first[nlin] = blocks;
    if (bits == 8) hipLaunchKernelGGL(wt_prep_kernel<8>, dim3(unsigned(blocks)), dim3(kThreads), 0, g->stream, a);
    else hipLaunchKernelGGL(wt_prep_kernel<4>, dim3(unsigned(blocks)), dim3(kThreads), 0, g->stream, a);
    return check_launch(g, "wt_prep");
}

bool bwd_fold_ok(int M, int N, int K, int G) {
    return M > 0 && M % 64 == 0 && N > 0 && N % 32 == 0 && K > 0 && K % 32 == 0 && G > 0 && G % 32 == 0 &&
           K % G == 0;
}

int gemm_bwd_fold(dgm_gpu* g, const int8_t* codesT, const float* scalesT, const float* dY, const float* X, float* dX,
                  float* dW, int M, int N, int K, int G, bool accumulate, const float* sg_gate, const float* sg_up) {
    if (!bwd_fold_ok(M, N, K, G) || !aligned(dY, 16) || !aligned(codesT, 8) || !aligned(scalesT, 16))
        return kNotFused;
    DxFoldArgs ax{};
    ax.dY = dY; ax.codesT = codesT; ax.scalesT = scalesT; ax.out = dX; ax.sg_gate = sg_gate; ax.sg_up = sg_up;
    ax.M = M; ax.N = N; ax.K = K; ax.G = G;
    GemmArgs aw{};
    aw.A = dY; aw.B = X; aw.out = dW;
    aw.M = M; aw.N = N; aw.K = K;
    aw.rows = N; aw.cols = K; aw.red = M;
    aw.G = 1; aw.groups = 0;
    aw.accumulate = accumulate;
    const int tm = M / 16, tk = K / 32;
    const int per_x = (tm * tk + 7) / 8;
    const int tn = int(ceil_div(N, 32)), tkw = int(ceil_div(K, 16));
    const int per_w = dW ? (tn * tkw + 7) / 8 : 0;   // no dW: the dX tiles alone
    hipLaunchKernelGGL(gemm_bwd_fold_pair_kernel, dim3(unsigned(per_x + per_w) * 8u), dim3(kThreads), 0, g->stream, ax,
                       tm, tk, per_x, aw, tn, tkw, per_w);
    return check_launch(g, "gemm_bwd_fold");
}

int gemm_check_sizes(dgm_gpu* g, const char* name, const dgm_GemmP* p, int bits) {
    return check_sizes(g, name, p, bits);
}

}  // namespace dgm
