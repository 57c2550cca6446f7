// One tile of the STE weight gradient dW[n, k] (=|+=) sum_m dY[m, n] * X[m, k]
// (metal/kernels.metal:270-283, 1014-1027), computed by a group of W waves.
// Shared by the GEMM library's dW and backward-pair kernels (W = 4) and by the
// DiT backward kernels that run dW tiles beside their own work (W = 16).
//
// A tile is 16 NP rows (n) x 16 columns (k); the W waves split M and load
// their operands straight into registers, CH 16-row chunks of loads issued
// before the first MFMA of a round. A lane reads dY[m, n0 + NP i .. + NP - 1]
// as one 8-byte (NP = 2) or 16-byte (NP = 4) load, so 16 lanes cover one or
// two whole 128-byte lines of a dY row; column e of the lane's NP feeds MFMA
// tile e (dW rows n0 + NP r + e). At step s a lane group q uses row m = m0 +
// q + 4 s. The W waves' partial tiles are added through LDS in a fixed
// order. Every dW element is the same chain of MFMAs over the same rows for
// any NP, CH and caller with the same W, so those results are bitwise equal.
#pragma once

#include <cstddef>
#include <cstdint>

namespace dgm_dw {

typedef float f32x4 __attribute__((ext_vector_type(4)));

struct DwTileArgs {
    const float* dY;   // [M, N]
    const float* X;    // [M, K]
    float* out;        // dW [N, K]
    int M, N, K;       // M % 64 == 0, N % NP == 0
    int accumulate;    // += instead of =
};

// Chunks per round of the 32 x 16 tile run beside other work.
constexpr int kPairCH = 2;
// Waves per tile of the tiles run beside other work: each wave's rows in as
// few rounds of loads as possible, so those tiles end before the work beside
// them (with four waves a 512-row tile takes four rounds).
constexpr int kHostedWaves = 16;
// 32 x 16 tiles (NP = 2) of a dW: along n, and in all.
inline int dw_tiles_n(const DwTileArgs& a) { return (a.N + 31) / 32; }
inline int dw_tiles(const DwTileArgs& a) { return dw_tiles_n(a) * ((a.K + 15) / 16); }

// Tile t (< tiles_n * tiles_k; `valid` false: no work) of a group whose waves
// are gw = 0..W-1 and threads gtid = 0..64 W - 1. part: the group's W NP KB of
// LDS. Wave gw takes the 16-row chunks [gw c / W, (gw + 1) c / W) of the
// c = M / 16.
// Every wave of the workgroup reaches the one __syncthreads, whatever its
// group's tile, so groups of one workgroup may hold different tiles or none.
// Lanes whose columns pass N load the last NP columns (N % NP == 0, so those
// lanes' own rows are all >= N) and are never stored.
template <int NP, int CH, int W = 4>
__device__ __forceinline__ void dw_tile(const DwTileArgs& a, bool valid, int t, int tiles_n, int gw, int gtid,
                                        float (*part)[NP][16][16]) {
    static_assert(NP == 2 || NP == 4, "2 or 4 columns per lane");
    static_assert(W == 4 || W == 16, "four or sixteen waves");
    const int lane = gtid & 63;
    const int r16 = lane & 15, q4 = lane >> 4;
    const int tk = valid ? t / tiles_n : 0, tn = valid ? t - tk * tiles_n : 0;
    const int n0 = tn * 16 * NP, k0 = tk * 16;
    const int M = a.M, N = a.N, K = a.K;
    f32x4 acc[NP];
#pragma unroll
    for (int e = 0; e < NP; ++e) acc[e] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    if (valid) {
        const int nc = min(n0 + NP * r16, N - NP);
        const int kc = min(k0 + r16, K - 1);
        const int nch = M >> 4;
        const int mb = 16 * (gw * nch / W), me = 16 * ((gw + 1) * nch / W);
        for (int r0 = mb; r0 < me; r0 += 16 * CH) {
            float av[CH][4][NP];
            float bv[CH][4];
#pragma unroll
            for (int c = 0; c < CH; ++c) {
                const int m0 = min(r0 + 16 * c, me - 16);   // past the range: re-read, not computed
#pragma unroll
                for (int s2 = 0; s2 < 4; ++s2) {
                    const int m = m0 + q4 + 4 * s2;
                    const float* src = a.dY + size_t(m) * N + nc;
                    if constexpr (NP == 4) {
                        const float4 v = *reinterpret_cast<const float4*>(src);
                        av[c][s2][0] = v.x; av[c][s2][1] = v.y; av[c][s2][2] = v.z; av[c][s2][3] = v.w;
                    } else {
                        const float2 v = *reinterpret_cast<const float2*>(src);
                        av[c][s2][0] = v.x; av[c][s2][1] = v.y;
                    }
                    bv[c][s2] = a.X[size_t(m) * K + kc];
                }
            }
            __builtin_amdgcn_sched_barrier(0);   // every load of the round before the first MFMA
#pragma unroll
            for (int c = 0; c < CH; ++c) {
                if (r0 + 16 * c >= me) continue;
#pragma unroll
                for (int s2 = 0; s2 < 4; ++s2)
#pragma unroll
                    for (int e = 0; e < NP; ++e)
                        acc[e] = __builtin_amdgcn_mfma_f32_16x16x4f32(av[c][s2][e], bv[c][s2], acc[e], 0, 0, 0);
            }
        }
        // acc[e][r]: dW row n0 + NP (4 q4 + r) + e, column k0 + r16.
#pragma unroll
        for (int r = 0; r < 4; ++r)
#pragma unroll
            for (int e = 0; e < NP; ++e) part[gw][e][4 * q4 + r][r16] = acc[e][r];
    }
    __syncthreads();
    if (!valid) return;
    for (int e = gtid; e < 16 * NP * 16; e += 64 * W) {
        const int il = e >> 4, j = e & 15;   // il: local dW row 0 .. 16 NP - 1
        const int i = n0 + il, k = k0 + j;
        if (i >= N || k >= K) continue;
        const int rr = il / NP, par = il - rr * NP;
        float v = part[0][par][rr][j];
#pragma unroll
        for (int w2 = 1; w2 < W; ++w2) v += part[w2][par][rr][j];
        float* o = a.out + size_t(i) * K + k;
        if (a.accumulate) *o += v;
        else *o = v;
    }
}

}  // namespace dgm_dw
