/*
 * CPU oracle for the group-quantized linear path — TEST INFRASTRUCTURE ONLY.
 *
 * This library is the checker, never the product. Only tests/, the smoke()
 * entry in __graft_entry__.py and the cpu_baseline leg of bench.py may load it.
 * The product path (diffusion-gpt-metal_amd/) never links, calls or falls back
 * to anything here.
 *
 * Every function restates a reference routine of githubpradeep/diffusion-gpt-metal
 * (paths relative to the reference root) in plain C, built with
 * -O2 -ffp-contract=off -fno-fast-math so that fp32 operations happen one at a
 * time in the reference's order, without FMA contraction or reassociation.
 *
 * Layout convention (the reference's): weights W[N,K] row-major, groups of G
 * along K inside each row, scales S[N, K/G] row-major, int8 codes Q8[N*K],
 * int4 codes Q4[N*K/2] with the even k in the low nibble.
 *
 * Pinning: see the header comment of oracle.c for how each function is pinned
 * by tests that do not restate its formula.
 */
#ifndef DGM_ORACLE_H
#define DGM_ORACLE_H
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* SplitMix64 stream + Box-Muller normal (src/GPU.swift:4-29). */
typedef struct { uint64_t state; } orc_rng;
void     orc_rng_init(orc_rng* r, uint64_t seed);
uint64_t orc_rng_next(orc_rng* r);
float    orc_rng_uniform(orc_rng* r);
float    orc_rng_normal(orc_rng* r);
/* n draws of normal()*std (Check.swift randn, GPT.swift:450-452 fillNormal). */
void     orc_fill_normal(orc_rng* r, float* out, int64_t n, float std);
/* Same stream, but returns the state after the call so callers can chain. */
uint64_t orc_normal_stream(uint64_t state, float* out, int64_t n, float std);

/* quant_code (kernels.metal:62-67, Check.swift:426-431). */
int  orc_quant_code(float w, float s, int lim);

/* cpuQuant (Check.swift:399-424 == kernels.metal:79-124). Quantizes
 * floor(cols/G) groups per row; codes of tail columns are left untouched and
 * scales are strided by floor(cols/G), as in the reference. bits = 8 writes
 * q8[rows*cols]; bits = 4 writes q4[rows*cols/2] (int4 needs an even G).
 * Returns 0, or -1 on a rejected shape. */
int  orc_quant(const float* w, int64_t rows, int64_t cols, int group, int bits,
               int8_t* q8, uint8_t* q4, float* scale);

/* dequant (Check.swift:433-458), generalised from its fixed G=8 to any G. */
int  orc_dequant(const void* q, const float* scale, int64_t rows, int64_t cols,
                 int group, int bits, float* out);

/* cpuGemmNT / cpuGemmDX / cpuGemmDW (Check.swift:460-494): sequential fp32,
 * bias first. bias may be NULL (the reference passes an empty array). */
void orc_gemm_nt(const float* x, const float* w, const float* bias, float* y,
                 int64_t M, int64_t N, int64_t K);
void orc_gemm_dx(const float* dy, const float* w, float* dx,
                 int64_t M, int64_t N, int64_t K);
void orc_gemm_dw(const float* dy, const float* x, float* dw,
                 int64_t M, int64_t N, int64_t K, int accumulate);

/* Metal kernel order for the quantized forward (kernels.metal:152-209):
 * per-group fp32 partial of code*x, then acc += partial*scale, bias last. */
int  orc_gemm_nt_q(const void* q, const float* scale, const float* x,
                   const float* bias, float* y, int64_t M, int64_t N, int64_t K,
                   int group, int bits);
/* Metal kernel order for the quantized dX (kernels.metal:226-268): each
 * weight dequantised (code*scale) before the multiply, n ascending. */
int  orc_gemm_dx_q(const void* q, const float* scale, const float* dy, float* dx,
                   int64_t M, int64_t N, int64_t K, int group, int bits);

/* ---- looped DiT block forward (src/DiT.swift:520-550) ------------------ */
void orc_rmsnorm_fwd(const float* x, float* y, float* rstd, const float* weight,
                     int64_t rows, int64_t cols, float eps);
void orc_rope_tables(int maxT, int dim, float theta, float* cosv, float* sinv);
void orc_rope_fwd(const float* x, float* y, const float* cosv, const float* sinv,
                  int B, int T, int H, int D);
void orc_repeat_heads(const float* src, float* dst, int B, int T, int H, int D);
void orc_attn_fwd(const float* q, const float* k, const float* v, float* scores,
                  float* probs, float* av, int B, int T, int H, int D, int causal);
void orc_swiglu_fwd(const float* gate, const float* up, float* y, int64_t n);
void orc_add(const float* a, const float* b, float* y, int64_t n);
void orc_mix(const float* a, const float* b, float* y, int64_t n, float ca, float cb);

/* The DiT loop body with every linear routed through the int8 (or int4)
 * group-quantised forward in the Metal kernel order. Weight codes/scales are
 * inputs (quantised once by the caller). x_io holds xs[0] on entry and
 * xs[loops] on exit. ws must hold orc_dit_workspace_floats() floats. */
typedef struct {
    int B, T, C, F, H, D, loops, group, bits;
    float eps, theta, mix;
} orc_dit_cfg;
int64_t orc_dit_workspace_floats(const orc_dit_cfg* c);
int orc_dit_forward(const orc_dit_cfg* c,
                    const void* qq, const float* sq, const void* qk, const float* sk,
                    const void* qv, const float* sv, const void* qo, const float* so,
                    const void* qg, const float* sg, const void* qu, const float* su,
                    const void* qd, const float* sd,
                    const float* n1, const float* n1b, const float* n2,
                    const float* n2b, const float* nf,
                    float* x_io, float* ws);

/* ---- training step: kernels.metal:285-295, 616-697, 749-802 ------------- */
void orc_adamw(float* w, const float* g, float* m, float* v, int64_t n, float lr, float b1,
               float b2, float eps, float wd, float invBC1, float invBC2);
float orc_reduce_sumsq(const float* x, int64_t n);
void orc_scale(float* x, int64_t n, float s);
int orc_embed(const uint32_t* tokens, const float* wte, const void* q, const float* scale,
              const float* wpe, float* y, int B, int T, int C, int group, int bits);
void orc_embed_bwd(const uint32_t* tokens, const float* dx, float* dwe, int B, int T, int C, int V);
void orc_pos_bwd(const float* dx, float* dwp, int B, int T, int C);
void orc_bias_grad(const float* dy, float* db, int64_t M, int64_t N);

/* ---- DiT block backward: kernels.metal:429-437, 508-612, 827-868, 891-949,
 * 970-1010; DiT.swift:558-626 ------------------------------------------- */
void orc_rms_bwd(const float* x, const float* rstd, const float* weight, const float* dy, float* dx,
                 float* dweight, int64_t rows, int64_t cols);
void orc_attn_bwd(const float* q, const float* k, const float* v, const float* probs, const float* dout,
                  float* dq, float* dk, float* dv, float* dprobs, float* dscores, int B, int T, int H, int D);
void orc_rope_bwd(const float* dy, float* dx, const float* cosv, const float* sinv, int B, int T, int H, int D);
void orc_swiglu_bwd(const float* gate, const float* up, const float* dy, float* dgate, float* dup, int64_t n);
void orc_sum_heads(const float* src, float* dst, int B, int T, int H, int D);
void orc_acc_scale(float* a, const float* b, int64_t n, float s);
/* One training step of the looped block: forward over cfg->loops loops saving
 * every loop's activations, then the backward of DiT.swift:566-626 (the loop
 * part). Linears: bits 32 uses w[i] (fp32 [N,K]); bits 8/4 run the forward on
 * the codes (Metal kernel order) and the STE dX through the dequantized codes.
 * x_io: xs[0] in, xs[loops] out. gy: dL/dxs[loops] in, dL/dxs[0] out.
 * gw[7] (+=, fp32 [N,K]) and gn[5] (+=, [C]) receive the weight gradients.
 * ws: orc_dit_train_floats(c) floats. */
int64_t orc_dit_train_floats(const orc_dit_cfg* c);
int orc_dit_train(const orc_dit_cfg* c, const float* const* w, const void* const* q,
                  const float* const* s, const float* const* norms, float* x_io, float* gy,
                  float* const* gw, float* const* gn, float* ws);

#ifdef __cplusplus
}
#endif
#endif
