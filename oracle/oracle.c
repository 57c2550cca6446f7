/*
 * CPU oracle for the group-quantized linear path — TEST INFRASTRUCTURE ONLY.
 *
 * Used solely as the checker by tests/, by __graft_entry__.smoke() and by the
 * cpu_baseline leg of bench.py. The product library never calls into it.
 * Build: oracle/build.sh (gcc -O2 -ffp-contract=off -fno-fast-math), which keeps
 * every fp32 operation separate and in source order, like the reference's
 * scalar Swift CPU path.
 *
 * How each function is pinned (tests/test_oracle.py), without restating it:
 *   orc_rng_*          SplitMix64 integer outputs against the published
 *                      splitmix64 reference values for seed 1234567; uniform()
 *                      against its closed form on those integers.
 *   orc_quant_code,    hand-derived known answers (power-of-two scales so the
 *   orc_quant          ties are exact: 2.5 -> 2, 3.5 -> 4, -2.5 -> -2; all-zero
 *                      group -> s = 1e-8f and code 0; nibble encodings
 *                      -7 -> 0x9, -1 -> 0xF, byte = lo | hi << 4), plus the
 *                      invariants |q| <= lim, the group arg-max codes to +-lim,
 *                      |q*s - w| <= s/2 (1 ulp slack), S == max(maxAbs/qmax,1e-8f),
 *                      and a float64 numpy brute force of the same definition.
 *   orc_dequant        q*s for hand-built codes; round trip |dequant - w| <= s/2.
 *   orc_gemm_*         float64 numpy matmul on the same dequantised weights
 *                      (tiny shapes: relative error <= 1e-6), and the identity
 *                      matrix / one-hot inputs that select a single row or column.
 *   DiT block pieces   rmsnorm: unit-RMS rows map to the weight; rope: norm
 *                      preservation per pair and the t = 0 identity; attention:
 *                      equal keys give the uniform average of v (the closed form
 *                      used by Check.swift:214-241); softmax rows sum to 1;
 *                      swiglu: silu(0) = 0 and float64 formula; block: float64
 *                      numpy restatement on a tiny config.
 *   orc_adamw          hand-derived exact steps (b1 = 1/2, b2 = 3/4, eps = 0:
 *                      the first update of a power-of-two gradient is exactly
 *                      sign(g)), pure decoupled decay at g = 0, and torch.optim
 *                      AdamW in float64 over several steps.
 *   orc_reduce_sumsq   exact integer-valued sums and a float64 sum.
 *   orc_embed*, orc_pos_bwd, orc_bias_grad
 *                      one-hot token tables that select rows, integer-valued
 *                      inputs whose sums are exact, and numpy scatter-add /
 *                      column sums in float64.
 * Nothing here is parity-unpinned.
 */
#include "oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

/* ---- RNG: src/GPU.swift:4-29 ------------------------------------------- */

void orc_rng_init(orc_rng* r, uint64_t seed) {
    /* GPU.swift:6-8: seed 0 is replaced by a fixed constant. */
    r->state = seed == 0 ? 0x123456789abcdef0ULL : seed;
}

uint64_t orc_rng_next(orc_rng* r) {
    /* GPU.swift:9-15 */
    r->state += 0x9E3779B97F4A7C15ULL;
    uint64_t z = r->state;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ULL;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBULL;
    return z ^ (z >> 31);
}

float orc_rng_uniform(orc_rng* r) {
    /* GPU.swift:16-19: top 24 bits, (x + 1) / 2^24, in fp32. */
    uint64_t x = orc_rng_next(r) >> 40;
    float xf = (float)x;
    return (xf + 1.0f) / 16777216.0f;
}

float orc_rng_normal(orc_rng* r) {
    /* GPU.swift:20-24. Swift's Float.pi is pi rounded toward zero (0x40490FDA).
     * logf/cosf come from the C library here and from Darwin in the reference,
     * so a draw may differ by an ulp; fixtures therefore store input bytes. */
    float u1 = orc_rng_uniform(r);
    if (u1 < 1e-7f) u1 = 1e-7f;
    float u2 = orc_rng_uniform(r);
    union { uint32_t u; float f; } pi = { 0x40490FDAu };
    float a = -2.0f * logf(u1);
    float b = 2.0f * pi.f;
    b = b * u2;
    return sqrtf(a) * cosf(b);
}

void orc_fill_normal(orc_rng* r, float* out, int64_t n, float std) {
    for (int64_t i = 0; i < n; ++i) out[i] = orc_rng_normal(r) * std;
}

uint64_t orc_normal_stream(uint64_t state, float* out, int64_t n, float std) {
    orc_rng r; r.state = state;
    orc_fill_normal(&r, out, n, std);
    return r.state;
}

/* ---- quantize: Check.swift:399-431, kernels.metal:62-124 ----------------- */

int orc_quant_code(float w, float s, int lim) {
    float r = rintf(w / s);         /* correctly rounded divide, ties to even */
    int q;
    if (r > 2147483520.0f) q = lim;          /* outside int range: clamps anyway */
    else if (r < -2147483520.0f) q = -lim;
    else q = (int)r;
    if (q > lim) q = lim;
    if (q < -lim) q = -lim;
    return q;
}

/* Shapes the GEMM/dequant side accepts: K % G == 0 (src/GPU.swift:229,247). */
static int shape_ok(int64_t rows, int64_t cols, int group, int bits) {
    if (rows < 0 || cols < 0 || group <= 0) return 0;
    if (bits != 8 && bits != 4) return 0;
    if (cols % group != 0) return 0;
    if (bits == 4 && (group % 2) != 0) return 0;
    return 1;
}

/* Shapes the quantizer accepts. cpuQuant / quant_i8 / quant_i4 do not require
 * cols % G == 0: they quantize floor(cols/G) groups per row, leave the codes
 * of the tail columns untouched and stride the scales by floor(cols/G)
 * (Check.swift:399-424, kernels.metal:86-98). An odd int4 group would read
 * past the group (the reference's GPTConfig.validate rejects it,
 * Params.swift:171), so it is rejected here. */
static int quant_shape_ok(int64_t rows, int64_t cols, int group, int bits) {
    if (rows < 0 || cols < 0 || group <= 0) return 0;
    if (bits != 8 && bits != 4) return 0;
    if (bits == 4 && (group % 2) != 0) return 0;
    return 1;
}

int orc_quant(const float* w, int64_t rows, int64_t cols, int group, int bits,
              int8_t* q8, uint8_t* q4, float* scale) {
    if (!quant_shape_ok(rows, cols, group, bits)) return -1;
    const float lim = bits == 4 ? 7.0f : 127.0f;
    const int ilim = (int)lim;
    const int64_t groups = cols / group;
    for (int64_t row = 0; row < rows; ++row) {
        for (int64_t g = 0; g < groups; ++g) {
            const int64_t base = row * cols + g * group;
            float maxAbs = 0.0f;
            for (int i = 0; i < group; ++i) {
                float a = fabsf(w[base + i]);
                maxAbs = a >= maxAbs ? a : maxAbs;   /* Swift max(x, y): y >= x ? y : x */
            }
            float d = maxAbs / lim;
            float s = 1e-8f >= d ? 1e-8f : d;
            scale[row * groups + g] = s;
            if (bits == 8) {
                for (int i = 0; i < group; ++i)
                    q8[base + i] = (int8_t)orc_quant_code(w[base + i], s, ilim);
            } else {
                for (int i = 0; i < group; i += 2) {
                    int c0 = orc_quant_code(w[base + i], s, ilim);
                    int c1 = orc_quant_code(w[base + i + 1], s, ilim);
                    q4[(base + i) >> 1] = (uint8_t)((c0 & 0xF) | ((c1 & 0xF) << 4));
                }
            }
        }
    }
    return 0;
}

/* Signed code at (row, col) of a packed matrix: Check.swift:450-452. */
static inline int code_at(const void* q, int64_t row, int64_t col, int64_t cols, int bits) {
    if (bits == 8) return ((const int8_t*)q)[row * cols + col];
    uint8_t b = ((const uint8_t*)q)[(row * cols + col) >> 1];
    int nib = (col & 1) ? (b >> 4) : (b & 0xF);
    return nib >= 8 ? nib - 16 : nib;
}

int orc_dequant(const void* q, const float* scale, int64_t rows, int64_t cols,
                int group, int bits, float* out) {
    if (!shape_ok(rows, cols, group, bits)) return -1;
    const int64_t groups = cols / group;
    for (int64_t n = 0; n < rows; ++n)
        for (int64_t k = 0; k < cols; ++k)
            out[n * cols + k] = (float)code_at(q, n, k, cols, bits) * scale[n * groups + k / group];
    return 0;
}

/* ---- fp32 GEMMs: Check.swift:460-494 ------------------------------------ */

void orc_gemm_nt(const float* x, const float* w, const float* bias, float* y,
                 int64_t M, int64_t N, int64_t K) {
    for (int64_t m = 0; m < M; ++m)
        for (int64_t n = 0; n < N; ++n) {
            float acc = bias ? bias[n] : 0.0f;
            for (int64_t k = 0; k < K; ++k) acc += x[m * K + k] * w[n * K + k];
            y[m * N + n] = acc;
        }
}

void orc_gemm_dx(const float* dy, const float* w, float* dx,
                 int64_t M, int64_t N, int64_t K) {
    for (int64_t m = 0; m < M; ++m)
        for (int64_t k = 0; k < K; ++k) {
            float acc = 0.0f;
            for (int64_t n = 0; n < N; ++n) acc += dy[m * N + n] * w[n * K + k];
            dx[m * K + k] = acc;
        }
}

void orc_gemm_dw(const float* dy, const float* x, float* dw,
                 int64_t M, int64_t N, int64_t K, int accumulate) {
    /* Check.swift:484-494 (overwrite) and kernels.metal:1014-1027 (+=). */
    for (int64_t n = 0; n < N; ++n)
        for (int64_t k = 0; k < K; ++k) {
            float acc = 0.0f;
            for (int64_t m = 0; m < M; ++m) acc += dy[m * N + n] * x[m * K + k];
            if (accumulate) dw[n * K + k] += acc;
            else dw[n * K + k] = acc;
        }
}

/* ---- Metal kernel orders: kernels.metal:152-209, 226-268 ----------------- */

int orc_gemm_nt_q(const void* q, const float* scale, const float* x,
                  const float* bias, float* y, int64_t M, int64_t N, int64_t K,
                  int group, int bits) {
    if (!shape_ok(N, K, group, bits)) return -1;
    const int64_t groups = K / group;
    for (int64_t m = 0; m < M; ++m)
        for (int64_t n = 0; n < N; ++n) {
            const float* xr = x + m * K;
            float acc = 0.0f;
            for (int64_t g = 0; g < groups; ++g) {
                float part = 0.0f;
                const int64_t base = g * group;
                if (bits == 8) {
                    for (int i = 0; i < group; ++i)
                        part += (float)code_at(q, n, base + i, K, 8) * xr[base + i];
                } else {
                    /* gemm_nt_i4 pairs two products before the add (kernels.metal:201-204). */
                    for (int i = 0; i < group; i += 2) {
                        float w0 = (float)code_at(q, n, base + i, K, 4);
                        float w1 = (float)code_at(q, n, base + i + 1, K, 4);
                        float p0 = w0 * xr[base + i];
                        float p1 = w1 * xr[base + i + 1];
                        part += p0 + p1;
                    }
                }
                acc += part * scale[n * groups + g];
            }
            if (bias) acc += bias[n];
            y[m * N + n] = acc;
        }
    return 0;
}

int orc_gemm_dx_q(const void* q, const float* scale, const float* dy, float* dx,
                  int64_t M, int64_t N, int64_t K, int group, int bits) {
    if (!shape_ok(N, K, group, bits)) return -1;
    const int64_t groups = K / group;
    for (int64_t m = 0; m < M; ++m)
        for (int64_t k = 0; k < K; ++k) {
            const int64_t g = k / group;
            float acc = 0.0f;
            for (int64_t n = 0; n < N; ++n) {
                float wv = (float)code_at(q, n, k, K, bits) * scale[n * groups + g];
                acc += dy[m * N + n] * wv;
            }
            dx[m * K + k] = acc;
        }
    return 0;
}

/* ---- DiT block pieces (kernels.metal line refs per function) ------------- */

void orc_rmsnorm_fwd(const float* x, float* y, float* rstd, const float* weight,
                     int64_t rows, int64_t cols, float eps) {
    /* kernels.metal:807-825 */
    for (int64_t r = 0; r < rows; ++r) {
        const float* xr = x + r * cols;
        float ss = 0.0f;
        for (int64_t c = 0; c < cols; ++c) ss += xr[c] * xr[c];
        ss /= (float)cols;
        float rs = 1.0f / sqrtf(ss + eps);
        if (rstd) rstd[r] = rs;
        float* yr = y + r * cols;
        for (int64_t c = 0; c < cols; ++c) yr[c] = (xr[c] * rs) * weight[c];
    }
}

void orc_rope_tables(int maxT, int dim, float theta, float* cosv, float* sinv) {
    /* src/Macro.swift:509-530 */
    int half = dim / 2;
    float* inv = (float*)malloc(sizeof(float) * (size_t)(half > 0 ? half : 1));
    for (int i = 0; i < half; ++i) {
        float e = (float)(2 * i) / (float)dim;
        inv[i] = powf(theta, -e);
    }
    for (int t = 0; t < maxT; ++t)
        for (int i = 0; i < half; ++i) {
            float f = (float)t * inv[i];
            float c = cosf(f), s = sinf(f);
            cosv[t * dim + i] = c; cosv[t * dim + i + half] = c;
            sinv[t * dim + i] = s; sinv[t * dim + i + half] = s;
        }
    free(inv);
}

void orc_rope_fwd(const float* x, float* y, const float* cosv, const float* sinv,
                  int B, int T, int H, int D) {
    /* kernels.metal:871-889: rotate-half, [B,T,H,D], tables [T,D]. */
    int64_t total = (int64_t)B * T * H * D;
    int mid = D >> 1;
    for (int64_t i = 0; i < total; ++i) {
        int d = (int)(i % D);
        int t = (int)((i / ((int64_t)H * D)) % T);
        float rot = d < mid ? -x[i + mid] : x[i - mid];
        float c = cosv[t * D + d], s = sinv[t * D + d];
        float a = x[i] * c, b = rot * s;
        y[i] = a + b;
    }
}

void orc_repeat_heads(const float* src, float* dst, int B, int T, int H, int D) {
    /* kernels.metal:980-993 */
    int64_t total = (int64_t)B * T * H * D;
    for (int64_t i = 0; i < total; ++i) {
        int d = (int)(i % D);
        int t = (int)((i / ((int64_t)H * D)) % T);
        int b = (int)(i / ((int64_t)T * H * D));
        dst[i] = src[((int64_t)b * T + t) * D + d];
    }
}

void orc_attn_fwd(const float* q, const float* k, const float* v, float* scores,
                  float* probs, float* av, int B, int T, int H, int D, int causal) {
    /* kernels.metal:443-506; scale = 1/sqrt(Float(D)) (GPU.swift attnP). */
    float scale = 1.0f / sqrtf((float)D);
    for (int b = 0; b < B; ++b)
        for (int h = 0; h < H; ++h)
            for (int t = 0; t < T; ++t) {
                float* srow = scores + (((int64_t)b * H + h) * T + t) * T;
                for (int s = 0; s < T; ++s) {
                    float acc = 0.0f;
                    for (int d = 0; d < D; ++d)
                        acc += q[(((int64_t)b * T + t) * H + h) * D + d] *
                               k[(((int64_t)b * T + s) * H + h) * D + d];
                    acc *= scale;
                    if (causal && s > t) acc = -1.0e30f;
                    srow[s] = acc;
                }
                float* prow = probs + (((int64_t)b * H + h) * T + t) * T;
                float mx = srow[0];
                for (int s = 1; s < T; ++s) mx = srow[s] > mx ? srow[s] : mx;
                float sum = 0.0f;
                for (int s = 0; s < T; ++s) sum += expf(srow[s] - mx);
                float inv = 1.0f / sum;
                for (int s = 0; s < T; ++s) prow[s] = expf(srow[s] - mx) * inv;
            }
    for (int b = 0; b < B; ++b)
        for (int t = 0; t < T; ++t)
            for (int h = 0; h < H; ++h)
                for (int d = 0; d < D; ++d) {
                    float acc = 0.0f;
                    for (int s = 0; s < T; ++s)
                        acc += probs[(((int64_t)b * H + h) * T + t) * T + s] *
                               v[(((int64_t)b * T + s) * H + h) * D + d];
                    av[(((int64_t)b * T + t) * H + h) * D + d] = acc;
                }
}

static float silu_sigmoid(float z) {
    /* kernels.metal:911-918 */
    if (z >= 0.0f) { float e = expf(-z); return 1.0f / (1.0f + e); }
    float e = expf(z);
    return e / (1.0f + e);
}

void orc_swiglu_fwd(const float* gate, const float* up, float* y, int64_t n) {
    /* kernels.metal:920-930 */
    for (int64_t i = 0; i < n; ++i) {
        float z = gate[i];
        float a = z * silu_sigmoid(z);
        y[i] = a * up[i];
    }
}

void orc_add(const float* a, const float* b, float* y, int64_t n) {
    for (int64_t i = 0; i < n; ++i) y[i] = a[i] + b[i];   /* kernels.metal:419-427 */
}

void orc_mix(const float* a, const float* b, float* y, int64_t n, float ca, float cb) {
    for (int64_t i = 0; i < n; ++i) {                      /* kernels.metal:951-959 */
        float p = ca * a[i], r = cb * b[i];
        y[i] = p + r;
    }
}

/* ---- DiT loop body: src/DiT.swift:520-550 -------------------------------- */

enum { W_LN1, W_QPRE, W_KPRE, W_VPRE, W_VFIRST, W_VMIX, W_Q, W_KROT, W_K, W_V,
       W_SCORES, W_PROBS, W_AV, W_ATTN, W_T1, W_MID, W_LN2, W_GATE, W_UP, W_SW,
       W_MLP, W_PRE, W_RSTD, W_COS, W_SIN, W_XN, W_COUNT };

static void dit_sizes(const orc_dit_cfg* c, int64_t* sz) {
    int64_t M = (int64_t)c->B * c->T, C = c->C, F = c->F, KV = c->D;
    int64_t att = (int64_t)c->B * c->H * c->T * c->T;
    int64_t s[W_COUNT] = { M * C, M * C, M * KV, M * KV, M * KV, M * KV, M * C, M * KV,
                           M * C, M * C, att, att, M * C, M * C, M * C, M * C, M * C,
                           M * F, M * F, M * F, M * C, M * C, M,
                           (int64_t)c->T * c->D, (int64_t)c->T * c->D, M * C };
    memcpy(sz, s, sizeof(s));
}

int64_t orc_dit_workspace_floats(const orc_dit_cfg* c) {
    int64_t sz[W_COUNT], total = 0;
    dit_sizes(c, sz);
    for (int i = 0; i < W_COUNT; ++i) total += sz[i];
    return total;
}

int orc_dit_forward(const orc_dit_cfg* c,
                    const void* qq, const float* sq, const void* qk, const float* sk,
                    const void* qv, const float* sv, const void* qo, const float* so,
                    const void* qg, const float* sg, const void* qu, const float* su,
                    const void* qd, const float* sd,
                    const float* n1, const float* n1b, const float* n2,
                    const float* n2b, const float* nf,
                    float* x_io, float* ws) {
    if (c->H * c->D != c->C || (c->D % 2) != 0) return -1;
    int64_t sz[W_COUNT];
    float* p[W_COUNT];
    dit_sizes(c, sz);
    float* cur = ws;
    for (int i = 0; i < W_COUNT; ++i) { p[i] = cur; cur += sz[i]; }
    const int B = c->B, T = c->T, H = c->H, D = c->D, G = c->group, bits = c->bits;
    const int64_t M = (int64_t)B * T, C = c->C, F = c->F, KV = D;
    orc_rope_tables(T, D, c->theta, p[W_COS], p[W_SIN]);
    float* x = x_io;
    float* xn = p[W_XN];
    for (int loop = 0; loop < c->loops; ++loop) {
        orc_rmsnorm_fwd(x, p[W_LN1], p[W_RSTD], n1, M, C, c->eps);
        if (orc_gemm_nt_q(qq, sq, p[W_LN1], NULL, p[W_QPRE], M, C, C, G, bits)) return -1;
        if (orc_gemm_nt_q(qk, sk, p[W_LN1], NULL, p[W_KPRE], M, KV, C, G, bits)) return -1;
        if (orc_gemm_nt_q(qv, sv, p[W_LN1], NULL, p[W_VPRE], M, KV, C, G, bits)) return -1;
        if (loop == 0) {
            memcpy(p[W_VFIRST], p[W_VPRE], sizeof(float) * (size_t)(M * KV));
            orc_repeat_heads(p[W_VPRE], p[W_V], B, T, H, D);
        } else {
            orc_mix(p[W_VPRE], p[W_VFIRST], p[W_VMIX], M * KV, 1.0f - c->mix, c->mix);
            orc_repeat_heads(p[W_VMIX], p[W_V], B, T, H, D);
        }
        orc_rope_fwd(p[W_QPRE], p[W_Q], p[W_COS], p[W_SIN], B, T, H, D);
        orc_rope_fwd(p[W_KPRE], p[W_KROT], p[W_COS], p[W_SIN], B, T, 1, D);
        orc_repeat_heads(p[W_KROT], p[W_K], B, T, H, D);
        orc_attn_fwd(p[W_Q], p[W_K], p[W_V], p[W_SCORES], p[W_PROBS], p[W_AV], B, T, H, D, 0);
        if (orc_gemm_nt_q(qo, so, p[W_AV], NULL, p[W_ATTN], M, C, C, G, bits)) return -1;
        orc_rmsnorm_fwd(p[W_ATTN], p[W_T1], p[W_RSTD], n1b, M, C, c->eps);
        orc_add(x, p[W_T1], p[W_MID], M * C);
        orc_rmsnorm_fwd(p[W_MID], p[W_LN2], p[W_RSTD], n2, M, C, c->eps);
        if (orc_gemm_nt_q(qg, sg, p[W_LN2], NULL, p[W_GATE], M, F, C, G, bits)) return -1;
        if (orc_gemm_nt_q(qu, su, p[W_LN2], NULL, p[W_UP], M, F, C, G, bits)) return -1;
        orc_swiglu_fwd(p[W_GATE], p[W_UP], p[W_SW], M * F);
        if (orc_gemm_nt_q(qd, sd, p[W_SW], NULL, p[W_MLP], M, C, F, G, bits)) return -1;
        orc_rmsnorm_fwd(p[W_MLP], p[W_T1], p[W_RSTD], n2b, M, C, c->eps);
        orc_add(p[W_MID], p[W_T1], p[W_PRE], M * C);
        orc_rmsnorm_fwd(p[W_PRE], xn, p[W_RSTD], nf, M, C, c->eps);
        memcpy(x, xn, sizeof(float) * (size_t)(M * C));
    }
    return 0;
}

/* ---- training step ------------------------------------------------------ */

/* adamw, kernels.metal:786-802 (each operation rounded separately). */
void orc_adamw(float* w, const float* g, float* m, float* v, int64_t n, float lr, float b1,
               float b2, float eps, float wd, float invBC1, float invBC2) {
    for (int64_t i = 0; i < n; ++i) {
        float gi = g[i];
        float mi = b1 * m[i] + (1.0f - b1) * gi;
        float vi = b2 * v[i] + (1.0f - b2) * gi * gi;
        m[i] = mi;
        v[i] = vi;
        float upd = (mi * invBC1) / (sqrtf(vi * invBC2) + eps);
        w[i] -= lr * (upd + wd * w[i]);
    }
}

/* reduce_sumsq, kernels.metal:749-768: 256 lane sums over i = lane (mod 256),
 * then the halving tree 128, 64, ..., 1. */
float orc_reduce_sumsq(const float* x, int64_t n) {
    float sh[256];
    for (int t = 0; t < 256; ++t) {
        float v = 0.0f;
        for (int64_t i = t; i < n; i += 256) {
            float a = x[i];
            v += a * a;
        }
        sh[t] = v;
    }
    for (int s = 128; s > 0; s >>= 1)
        for (int t = 0; t < s; ++t) sh[t] += sh[t + s];
    return sh[0];
}

/* scale_f, kernels.metal:778-784. */
void orc_scale(float* x, int64_t n, float s) {
    for (int64_t i = 0; i < n; ++i) x[i] *= s;
}

/* embed_f32 / embed_i8 / embed_i4, kernels.metal:616-663: the dequantized
 * table entry code * scale is rounded, then wpe is added. bits 32 reads wte. */
int orc_embed(const uint32_t* tokens, const float* wte, const void* q, const float* scale,
              const float* wpe, float* y, int B, int T, int C, int group, int bits) {
    if (bits != 32 && !shape_ok(1, C, group, bits)) return -1;
    const int groups = bits == 32 ? 0 : C / group;
    for (int bt = 0; bt < B * T; ++bt) {
        const int t = bt % T;
        const int64_t tok = tokens[bt];
        for (int c = 0; c < C; ++c) {
            float e;
            if (bits == 32) e = wte[tok * C + c];
            else e = (float)code_at(q, tok, c, C, bits) * scale[tok * groups + c / group];
            y[(int64_t)bt * C + c] = e + wpe[(int64_t)t * C + c];
        }
    }
    return 0;
}

/* embed_bwd, kernels.metal:665-682: for each (v, c) a sum from 0 over bt in
 * increasing order, then added to dwe. */
void orc_embed_bwd(const uint32_t* tokens, const float* dx, float* dwe, int B, int T, int C, int V) {
    const int BT = B * T;
    for (int v = 0; v < V; ++v)
        for (int c = 0; c < C; ++c) {
            float sum = 0.0f;
            for (int bt = 0; bt < BT; ++bt)
                if (tokens[bt] == (uint32_t)v) sum += dx[(int64_t)bt * C + c];
            dwe[(int64_t)v * C + c] += sum;
        }
}

/* pos_bwd, kernels.metal:684-697. */
void orc_pos_bwd(const float* dx, float* dwp, int B, int T, int C) {
    for (int t = 0; t < T; ++t)
        for (int c = 0; c < C; ++c) {
            float sum = 0.0f;
            for (int b = 0; b < B; ++b) sum += dx[((int64_t)b * T + t) * C + c];
            dwp[(int64_t)t * C + c] = sum;
        }
}

/* bias_grad, kernels.metal:285-295. */
void orc_bias_grad(const float* dy, float* db, int64_t M, int64_t N) {
    for (int64_t n = 0; n < N; ++n) {
        float acc = 0.0f;
        for (int64_t m = 0; m < M; ++m) acc += dy[m * N + n];
        db[n] = acc;
    }
}

/* ---- DiT block backward ------------------------------------------------- */

/* rmsnorm_bwd_dx + rmsnorm_bwd_dw, kernels.metal:827-868 (GPU.rmsBwd,
 * GPU.swift:369-373): dweight accumulates. */
void orc_rms_bwd(const float* x, const float* rstd, const float* weight, const float* dy, float* dx,
                 float* dweight, int64_t rows, int64_t cols) {
    for (int64_t r = 0; r < rows; ++r) {
        const float rs = rstd[r];
        float meanDyX = 0.0f;
        for (int64_t c = 0; c < cols; ++c) {
            float dyhat = dy[r * cols + c] * weight[c];
            meanDyX += dyhat * x[r * cols + c];
        }
        meanDyX /= (float)cols;
        float rs3 = rs * rs * rs;
        for (int64_t c = 0; c < cols; ++c) {
            float dyhat = dy[r * cols + c] * weight[c];
            dx[r * cols + c] = rs * dyhat - x[r * cols + c] * rs3 * meanDyX;
        }
    }
    for (int64_t c = 0; c < cols; ++c) {
        float dg = 0.0f;
        for (int64_t r = 0; r < rows; ++r) dg += dy[r * cols + c] * x[r * cols + c] * rstd[r];
        dweight[c] += dg;
    }
}

/* attn_bwd_dv / attn_bwd_dp / attn_softmax_bwd / attn_bwd_dq / attn_bwd_dk,
 * kernels.metal:508-612, in GPU.attnBwd's order (GPU.swift:312-322). */
void orc_attn_bwd(const float* q, const float* k, const float* v, const float* probs, const float* dout,
                  float* dq, float* dk, float* dv, float* dprobs, float* dscores, int B, int T, int H, int D) {
    const float scale = 1.0f / sqrtf((float)D);
#define QI(b, t, h, d) ((((int64_t)(b) * T + (t)) * H + (h)) * D + (d))
#define PI(b, h, t, s) ((((int64_t)(b) * H + (h)) * T + (t)) * T + (s))
    for (int b = 0; b < B; ++b)
        for (int s = 0; s < T; ++s)
            for (int h = 0; h < H; ++h)
                for (int d = 0; d < D; ++d) {
                    float acc = 0.0f;
                    for (int t = 0; t < T; ++t) acc += probs[PI(b, h, t, s)] * dout[QI(b, t, h, d)];
                    dv[QI(b, s, h, d)] = acc;
                }
    for (int b = 0; b < B; ++b)
        for (int h = 0; h < H; ++h)
            for (int t = 0; t < T; ++t)
                for (int s = 0; s < T; ++s) {
                    float acc = 0.0f;
                    for (int d = 0; d < D; ++d) acc += dout[QI(b, t, h, d)] * v[QI(b, s, h, d)];
                    dprobs[PI(b, h, t, s)] = acc;
                }
    for (int64_t row = 0; row < (int64_t)B * H * T; ++row) {
        const float* pr = probs + row * T;
        const float* g = dprobs + row * T;
        float* o = dscores + row * T;
        float dot = 0.0f;
        for (int i = 0; i < T; ++i) dot += g[i] * pr[i];
        for (int i = 0; i < T; ++i) o[i] = pr[i] * (g[i] - dot);
    }
    for (int b = 0; b < B; ++b)
        for (int t = 0; t < T; ++t)
            for (int h = 0; h < H; ++h)
                for (int d = 0; d < D; ++d) {
                    float acc = 0.0f;
                    for (int s = 0; s < T; ++s) acc += dscores[PI(b, h, t, s)] * k[QI(b, s, h, d)];
                    dq[QI(b, t, h, d)] = acc * scale;
                }
    for (int b = 0; b < B; ++b)
        for (int s = 0; s < T; ++s)
            for (int h = 0; h < H; ++h)
                for (int d = 0; d < D; ++d) {
                    float acc = 0.0f;
                    for (int t = 0; t < T; ++t) acc += dscores[PI(b, h, t, s)] * q[QI(b, t, h, d)];
                    dk[QI(b, s, h, d)] = acc * scale;
                }
#undef QI
#undef PI
}

/* rope_bwd, kernels.metal:891-909. */
void orc_rope_bwd(const float* dy, float* dx, const float* cosv, const float* sinv, int B, int T, int H, int D) {
    const int64_t total = (int64_t)B * T * H * D;
    const int mid = D >> 1;
    for (int64_t i = 0; i < total; ++i) {
        int d = (int)(i % D);
        int t = (int)((i / ((int64_t)H * D)) % T);
        float c = cosv[t * D + d], s = sinv[t * D + d];
        if (d < mid) dx[i] = dy[i] * c + dy[i + mid] * s;
        else dx[i] = dy[i] * c - dy[i - mid] * s;
    }
}

/* swiglu_bwd, kernels.metal:932-949. */
void orc_swiglu_bwd(const float* gate, const float* up, const float* dy, float* dgate, float* dup, int64_t n) {
    for (int64_t i = 0; i < n; ++i) {
        float z = gate[i];
        float s = silu_sigmoid(z);
        float silu = z * s;
        float siluP = s * (1.0f + z * (1.0f - s));
        float g = dy[i];
        dgate[i] = siluP * up[i] * g;
        dup[i] = silu * g;
    }
}

/* sum_heads, kernels.metal:995-1010. */
void orc_sum_heads(const float* src, float* dst, int B, int T, int H, int D) {
    for (int64_t i = 0; i < (int64_t)B * T * D; ++i) {
        int d = (int)(i % D);
        int t = (int)((i / D) % T);
        int b = (int)(i / ((int64_t)T * D));
        float acc = 0.0f;
        for (int h = 0; h < H; ++h) acc += src[(((int64_t)b * T + t) * H + h) * D + d];
        dst[i] = acc;
    }
}

/* acc_scale_f, kernels.metal:970-977 (acc_f, 429-436, is s = 1 without the
 * product: see orc_dit_train). */
void orc_acc_scale(float* a, const float* b, int64_t n, float s) {
    for (int64_t i = 0; i < n; ++i) a[i] += s * b[i];
}

static void acc_f(float* a, const float* b, int64_t n) {
    for (int64_t i = 0; i < n; ++i) a[i] += b[i];
}

/* Saved activations of one loop (DiT.swift's Acts) and the step's scratch. */
enum { A_X, A_LN1, A_R1, A_Q, A_K, A_V, A_PROBS, A_AV, A_ATTN, A_R1B, A_MID, A_LN2, A_R2,
       A_GATE, A_UP, A_SW, A_MLP, A_R2B, A_PRE, A_RF, A_COUNT };
enum { S_QPRE, S_KPRE, S_VPRE, S_VFIRST, S_VMIX, S_KROT, S_SCORES, S_T1, S_T2, S_DLN, S_DSW, S_DG,
       S_DU, S_DAV, S_DQ, S_DK, S_DV, S_DPROBS, S_DK1, S_DV1, S_DVPRE, S_DFIRST, S_COS, S_SIN,
       S_COUNT };

static void train_sizes(const orc_dit_cfg* c, int64_t* a, int64_t* sc) {
    int64_t M = (int64_t)c->B * c->T, C = c->C, F = c->F, KV = c->D;
    int64_t att = (int64_t)c->B * c->H * c->T * c->T;
    int64_t av[A_COUNT] = { M * C, M * C, M, M * C, M * C, M * C, att, M * C, M * C, M, M * C, M * C, M,
                            M * F, M * F, M * F, M * C, M, M * C, M };
    int64_t sv[S_COUNT] = { M * C, M * KV, M * KV, M * KV, M * KV, M * KV, att, M * C, M * C, M * C, M * F,
                            M * F, M * F, M * C, M * C, M * C, M * C, att, M * KV, M * KV, M * KV, M * KV,
                            (int64_t)c->T * c->D, (int64_t)c->T * c->D };
    memcpy(a, av, sizeof(av));
    memcpy(sc, sv, sizeof(sv));
}

int64_t orc_dit_train_floats(const orc_dit_cfg* c) {
    int64_t a[A_COUNT], sc[S_COUNT], per = 0, tot = 0;
    train_sizes(c, a, sc);
    for (int i = 0; i < A_COUNT; ++i) per += a[i];
    for (int i = 0; i < S_COUNT; ++i) tot += sc[i];
    return per * (c->loops > 0 ? c->loops : 1) + tot;
}

static int lin_fwd(const orc_dit_cfg* c, int i, const float* const* w, const void* const* q,
                   const float* const* s, const float* x, float* y, int64_t M, int64_t N, int64_t K) {
    if (c->bits == 32) { orc_gemm_nt(x, w[i], NULL, y, M, N, K); return 0; }
    return orc_gemm_nt_q(q[i], s[i], x, NULL, y, M, N, K, c->group, c->bits);
}

static int lin_dx(const orc_dit_cfg* c, int i, const float* const* w, const void* const* q,
                  const float* const* s, const float* dy, float* dx, int64_t M, int64_t N, int64_t K) {
    if (c->bits == 32) { orc_gemm_dx(dy, w[i], dx, M, N, K); return 0; }
    return orc_gemm_dx_q(q[i], s[i], dy, dx, M, N, K, c->group, c->bits);
}

int orc_dit_train(const orc_dit_cfg* c, const float* const* w, const void* const* q,
                  const float* const* s, const float* const* norms, float* x_io, float* gy,
                  float* const* gw, float* const* gn, float* ws) {
    if (c->H * c->D != c->C || (c->D % 2) != 0) return -1;
    enum { WQ, WK, WV, WO, WG, WU, WD };
    const float *n1 = norms[0], *n1b = norms[1], *n2 = norms[2], *n2b = norms[3], *nf = norms[4];
    int64_t asz[A_COUNT], ssz[S_COUNT];
    train_sizes(c, asz, ssz);
    const int L = c->loops;
    float* cur = ws;
    float* A[64][A_COUNT];
    float* S[S_COUNT];
    if (L > 64) return -1;
    for (int l = 0; l < L; ++l)
        for (int i = 0; i < A_COUNT; ++i) { A[l][i] = cur; cur += asz[i]; }
    for (int i = 0; i < S_COUNT; ++i) { S[i] = cur; cur += ssz[i]; }
    const int B = c->B, T = c->T, H = c->H, D = c->D;
    const int64_t M = (int64_t)B * T, C = c->C, F = c->F, KV = D, nC = M * C, nKV = M * KV;
    const float mix = c->mix;
    orc_rope_tables(T, D, c->theta, S[S_COS], S[S_SIN]);
    /* forward, DiT.swift:520-550, saving each loop's activations */
    for (int l = 0; l < L; ++l) {
        float** a = A[l];
        if (l == 0) memcpy(a[A_X], x_io, sizeof(float) * (size_t)nC);
        orc_rmsnorm_fwd(a[A_X], a[A_LN1], a[A_R1], n1, M, C, c->eps);
        if (lin_fwd(c, WQ, w, q, s, a[A_LN1], S[S_QPRE], M, C, C)) return -1;
        if (lin_fwd(c, WK, w, q, s, a[A_LN1], S[S_KPRE], M, KV, C)) return -1;
        if (lin_fwd(c, WV, w, q, s, a[A_LN1], S[S_VPRE], M, KV, C)) return -1;
        if (l == 0) {
            memcpy(S[S_VFIRST], S[S_VPRE], sizeof(float) * (size_t)nKV);
            orc_repeat_heads(S[S_VPRE], a[A_V], B, T, H, D);
        } else {
            orc_mix(S[S_VPRE], S[S_VFIRST], S[S_VMIX], nKV, 1.0f - mix, mix);
            orc_repeat_heads(S[S_VMIX], a[A_V], B, T, H, D);
        }
        orc_rope_fwd(S[S_QPRE], a[A_Q], S[S_COS], S[S_SIN], B, T, H, D);
        orc_rope_fwd(S[S_KPRE], S[S_KROT], S[S_COS], S[S_SIN], B, T, 1, D);
        orc_repeat_heads(S[S_KROT], a[A_K], B, T, H, D);
        orc_attn_fwd(a[A_Q], a[A_K], a[A_V], S[S_SCORES], a[A_PROBS], a[A_AV], B, T, H, D, 0);
        if (lin_fwd(c, WO, w, q, s, a[A_AV], a[A_ATTN], M, C, C)) return -1;
        orc_rmsnorm_fwd(a[A_ATTN], S[S_T1], a[A_R1B], n1b, M, C, c->eps);
        orc_add(a[A_X], S[S_T1], a[A_MID], nC);
        orc_rmsnorm_fwd(a[A_MID], a[A_LN2], a[A_R2], n2, M, C, c->eps);
        if (lin_fwd(c, WG, w, q, s, a[A_LN2], a[A_GATE], M, F, C)) return -1;
        if (lin_fwd(c, WU, w, q, s, a[A_LN2], a[A_UP], M, F, C)) return -1;
        orc_swiglu_fwd(a[A_GATE], a[A_UP], a[A_SW], M * F);
        if (lin_fwd(c, WD, w, q, s, a[A_SW], a[A_MLP], M, C, F)) return -1;
        orc_rmsnorm_fwd(a[A_MLP], S[S_T1], a[A_R2B], n2b, M, C, c->eps);
        orc_add(a[A_MID], S[S_T1], a[A_PRE], nC);
        float* xn = l + 1 < L ? A[l + 1][A_X] : x_io;
        orc_rmsnorm_fwd(a[A_PRE], xn, a[A_RF], nf, M, C, c->eps);
    }
    /* backward, DiT.swift:566-626 (the loop part; gy plays gx) */
    float *t1 = S[S_T1], *t2 = S[S_T2], *dln = S[S_DLN];
    memset(S[S_DFIRST], 0, sizeof(float) * (size_t)nKV);
    for (int l = L - 1; l >= 0; --l) {
        float** a = A[l];
        orc_rms_bwd(a[A_PRE], a[A_RF], nf, gy, t1, gn[4], M, C);
        orc_rms_bwd(a[A_MLP], a[A_R2B], n2b, t1, t2, gn[3], M, C);
        orc_gemm_dw(t2, a[A_SW], gw[WD], M, C, F, 1);
        if (lin_dx(c, WD, w, q, s, t2, S[S_DSW], M, C, F)) return -1;
        orc_swiglu_bwd(a[A_GATE], a[A_UP], S[S_DSW], S[S_DG], S[S_DU], M * F);
        orc_gemm_dw(S[S_DG], a[A_LN2], gw[WG], M, F, C, 1);
        if (lin_dx(c, WG, w, q, s, S[S_DG], t2, M, F, C)) return -1;
        orc_gemm_dw(S[S_DU], a[A_LN2], gw[WU], M, F, C, 1);
        if (lin_dx(c, WU, w, q, s, S[S_DU], dln, M, F, C)) return -1;
        acc_f(t2, dln, nC);
        orc_rms_bwd(a[A_MID], a[A_R2], n2, t2, dln, gn[2], M, C);
        acc_f(t1, dln, nC);
        orc_rms_bwd(a[A_ATTN], a[A_R1B], n1b, t1, t2, gn[1], M, C);
        orc_gemm_dw(t2, a[A_AV], gw[WO], M, C, C, 1);
        if (lin_dx(c, WO, w, q, s, t2, S[S_DAV], M, C, C)) return -1;
        orc_attn_bwd(a[A_Q], a[A_K], a[A_V], a[A_PROBS], S[S_DAV], S[S_DQ], S[S_DK], S[S_DV],
                     S[S_DPROBS], S[S_SCORES], B, T, H, D);
        orc_sum_heads(S[S_DK], S[S_DK1], B, T, H, D);
        orc_sum_heads(S[S_DV], S[S_DV1], B, T, H, D);
        orc_rope_bwd(S[S_DQ], S[S_QPRE], S[S_COS], S[S_SIN], B, T, H, D);
        orc_rope_bwd(S[S_DK1], S[S_KPRE], S[S_COS], S[S_SIN], B, T, 1, D);
        if (l == 0) {
            memcpy(S[S_DVPRE], S[S_DV1], sizeof(float) * (size_t)nKV);
            acc_f(S[S_DVPRE], S[S_DFIRST], nKV);
        } else {
            orc_mix(S[S_DV1], S[S_DV1], S[S_DVPRE], nKV, 1.0f - mix, 0.0f);
            orc_acc_scale(S[S_DFIRST], S[S_DV1], nKV, mix);
        }
        orc_gemm_dw(S[S_QPRE], a[A_LN1], gw[WQ], M, C, C, 1);
        if (lin_dx(c, WQ, w, q, s, S[S_QPRE], t2, M, C, C)) return -1;
        orc_gemm_dw(S[S_KPRE], a[A_LN1], gw[WK], M, KV, C, 1);
        if (lin_dx(c, WK, w, q, s, S[S_KPRE], dln, M, KV, C)) return -1;
        acc_f(t2, dln, nC);
        orc_gemm_dw(S[S_DVPRE], a[A_LN1], gw[WV], M, KV, C, 1);
        if (lin_dx(c, WV, w, q, s, S[S_DVPRE], dln, M, KV, C)) return -1;
        acc_f(t2, dln, nC);
        orc_rms_bwd(a[A_X], a[A_R1], n1, t2, dln, gn[0], M, C);
        acc_f(t1, dln, nC);
        memcpy(gy, t1, sizeof(float) * (size_t)nC);
    }
    return 0;
}
