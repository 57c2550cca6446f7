/*
 * dgm_quant.h — C ABI of the MI355X (gfx950) group-quantized linear path.
 *
 * Drop-in for the reference's quantize / group-quant GEMM / STE backward
 * dispatch surface (githubpradeep/diffusion-gpt-metal, paths relative to the
 * reference root). Plain pointers and sizes only: every buffer is device
 * memory owned by the caller, nothing here allocates caller-visible memory,
 * and every call returns an int status (0 = DGM_OK).
 *
 * Layouts are the reference's, unchanged:
 *   W   fp32 master weights [N, K] row-major (output rows x input cols)
 *   Q8  int8 codes [N*K], one byte per weight, codes in [-127, 127]
 *   Q4  int4 codes [N*K/2] bytes, two signed nibbles per byte, even k in the
 *       low nibble, codes in [-7, 7]
 *   S   fp32 scales [N, K/G] row-major, one per (row, group of G along K)
 *   X [M,K], Y [M,N], dY [M,N], dX [M,K], dW [N,K]: fp32 row-major
 *
 * Ordering: one HIP stream per context. Calls are enqueued in issue order
 * (the reference puts a full buffer barrier between dispatches,
 * src/GPU.swift:182-198, which an in-order stream already gives).
 */
#ifndef DGM_QUANT_H
#define DGM_QUANT_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- status codes -------------------------------------------------------- */
#define DGM_OK              0
#define DGM_ERR_ARG         1   /* null pointer / negative size / bad enum     */
#define DGM_ERR_SHAPE       2   /* a reference precondition failed, e.g.
                                   K % qGroup != 0 (src/GPU.swift:229,247) or
                                   odd group for int4 (src/Params.swift:171)  */
#define DGM_ERR_NOT_BEGUN   3   /* dispatch outside begin()/end()
                                   (src/GPU.swift:183)                        */
#define DGM_ERR_HIP         4   /* HIP launch or execution error              */
#define DGM_ERR_BITS        5   /* bits not in {32, 8, 4} (src/GPU.swift:241) */
#define DGM_ERR_UNSUPPORTED 6   /* size beyond what a kernel indexes (2^31)   */

/* ---- math modes (dgm_set_math) ------------------------------------------ */
/* FP32 (default): every result is within max relative error 1e-5 of the
 * float64 product. Quantized forwards of a few rows (M <= 4, and up to
 * M = 16 for weights large enough to split K over the CUs) run on int8 MFMA
 * over an exact split of the activations into four int8 pieces against a
 * power of two per row and k-range (2^-27 of its maximum); other forwards up
 * to M = 64 on f16 MFMA over two f16 pieces per activation against a power
 * of two per (row, 128-k block) (2^-22 of each element); the rest accumulate
 * fp32 products of fp32 operands.
 * BF16: the int8-piece kernels take two pieces (up to M = 8 when K is
 * split); otherwise up to M = 64, int4 codes
 * meet bf16(x) and int8 codes one f16 piece; larger M (with K % 128 == 0 and
 * qGroup % 32 == 0) runs on bf16 MFMA with activations rounded to bf16 and
 * weights dequantized to bf16 in LDS, fp32 accumulate. Max relative error
 * <= 1e-2. dX and dW are fp32 in both modes. */
#define DGM_MATH_FP32 0
#define DGM_MATH_BF16 1

/* ---- parameter blocks: src/Params.swift:7-23, metal/kernels.metal:22-29 -- */
typedef struct dgm_GemmP {
    uint32_t M, N, K, hasBias, qGroup, pad0, pad1, pad2;
} dgm_GemmP;                                   /* 32 bytes (src/GPU.swift:455) */

typedef struct dgm_QuantP {
    uint32_t rows, cols;
    float qmax;                                /* 127 (int8) or 7 (int4)       */
    uint32_t qGroup;
} dgm_QuantP;                                  /* 16 bytes (src/GPU.swift:456) */

/* ---- context: src/GPU.swift:91-198 (class GPU) --------------------------- */
typedef struct dgm_gpu dgm_gpu;

/* GPU.init (src/GPU.swift:118-156): binds the current HIP device and creates
 * the context's own stream. */
int dgm_gpu_create(dgm_gpu** out);
/* Waits for the work queued on the context's own stream and on every stream
 * it was set to (so those must still exist; after more than 16 distinct
 * streams, for the whole device), then frees its workspace. Graphs captured
 * from calls on the context read that workspace: they must not be replayed
 * after the context is destroyed. Other streams are not synchronized, so a
 * capture in progress elsewhere is undisturbed. */
void dgm_gpu_destroy(dgm_gpu* g);
/* Use a caller-owned stream (e.g. a framework's current stream) instead of the
 * context's own; NULL restores the context's stream. */
int dgm_gpu_set_stream(dgm_gpu* g, void* hip_stream);
void* dgm_gpu_stream(const dgm_gpu* g);
int dgm_set_math(dgm_gpu* g, int mode);
int dgm_get_math(const dgm_gpu* g);

/* GPU.begin (src/GPU.swift:158-166): opens a dispatch region. */
int dgm_begin(dgm_gpu* g);
/* GPU.end (src/GPU.swift:168-180): waits for the region's work and returns the
 * first error of the region (the reference prints it with lastKernel and
 * exits; callers turn a nonzero status into their own fatal error). This
 * includes DGM_ERR_HIP when a decode kernel of the region gave up one of its
 * bounded in-workgroup waits, whose results are then not valid (the flag is
 * per device: with several contexts on one device, the first end() that
 * follows reports it). */
int dgm_end(dgm_gpu* g);
/* GPU.lastKernel (src/GPU.swift:99): name of the last dispatched kernel. */
const char* dgm_last_kernel(const dgm_gpu* g);
/* Human-readable text of the context's last error ("" when none). */
const char* dgm_last_error(const dgm_gpu* g);

/* ---- kernel-level entry points: buffer slot order of metal/kernels.metal -- */

/* quant_i8 (metal/kernels.metal:79-98): W f32 -> Q i8 codes, S f32 scales. */
int dgm_quant_i8(dgm_gpu* g, const float* W, int8_t* Q, float* scale,
                 const dgm_QuantP* p);
/* quant_i4 (metal/kernels.metal:100-124): W f32 -> packed nibbles, S. */
int dgm_quant_i4(dgm_gpu* g, const float* W, uint8_t* Q, float* scale,
                 const dgm_QuantP* p);

/* gemm_nt_f32 (metal/kernels.metal:128-150): Y = X W^T (+bias). */
int dgm_gemm_nt_f32(dgm_gpu* g, const float* W, const float* X,
                    const float* bias, float* Y, const dgm_GemmP* p);
/* gemm_nt_i8 (metal/kernels.metal:152-178): Y = X dequant(Q8,S)^T (+bias). */
int dgm_gemm_nt_i8(dgm_gpu* g, const int8_t* W, const float* scale,
                   const float* X, const float* bias, float* Y,
                   const dgm_GemmP* p);
/* gemm_nt_i4 (metal/kernels.metal:180-209): Y = X dequant(Q4,S)^T (+bias). */
int dgm_gemm_nt_i4(dgm_gpu* g, const uint8_t* W, const float* scale,
                   const float* X, const float* bias, float* Y,
                   const dgm_GemmP* p);

/* gemm_dx_f32 (metal/kernels.metal:211-224): dX = dY W. */
int dgm_gemm_dx_f32(dgm_gpu* g, const float* W, const float* dY, float* dX,
                    const dgm_GemmP* p);
/* gemm_dx_i8 (metal/kernels.metal:226-246): STE dX = dY dequant(Q8,S). */
int dgm_gemm_dx_i8(dgm_gpu* g, const int8_t* W, const float* scale,
                   const float* dY, float* dX, const dgm_GemmP* p);
/* gemm_dx_i4 (metal/kernels.metal:248-268): STE dX = dY dequant(Q4,S). */
int dgm_gemm_dx_i4(dgm_gpu* g, const uint8_t* W, const float* scale,
                   const float* dY, float* dX, const dgm_GemmP* p);

/* gemm_dw (metal/kernels.metal:270-283): dW = dY^T X, overwrite. */
int dgm_gemm_dw(dgm_gpu* g, const float* dY, const float* X, float* dW,
                const dgm_GemmP* p);
/* gemm_dw_acc (metal/kernels.metal:1014-1027): dW += dY^T X. */
int dgm_gemm_dw_acc(dgm_gpu* g, const float* dY, const float* X, float* dW,
                    const dgm_GemmP* p);

/* ---- host call surface: src/GPU.swift:220-272 ----------------------------
 * Same names and argument meaning as the Swift wrappers. Sizes are Swift Int
 * (int64_t). q is int8_t* for bits 8, uint8_t* for bits 4; w is read only
 * when bits == 32. bias may be NULL (the reference binds a dummy buffer and
 * sets hasBias = 0). */

/* GPU.quantize (src/GPU.swift:220-225): qmax = 7 for bits 4, else 127. */
int dgm_quantize(dgm_gpu* g, const float* w, void* q, float* scale,
                 int64_t rows, int64_t cols, int64_t bits, int64_t qGroup);
/* GPU.gemmNT (src/GPU.swift:227-243). */
int dgm_gemmNT(dgm_gpu* g, int64_t bits, const float* w, const void* q,
               const float* scale, const float* x, const float* bias, float* y,
               int64_t M, int64_t N, int64_t K, int64_t qGroup);
/* No counterpart in the reference: dgm_gemmNT for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc). Same arguments, kernels and results
 * (bitwise) as dgm_gemmNT, but every staging buffer (the decode kernels'
 * activation pieces, the bf16 copy of X of the reduced-precision prefill
 * path) comes from a static device scratch of DGM_NOALLOC_SCRATCH_BYTES per
 * GPU, held from library load until the process ends; nothing is allocated.
 * A call that would need more scratch returns DGM_ERR_UNSUPPORTED before
 * launching anything (dgm_gemmNT_workspace_bound gives the most a call can
 * need: at most 260 * K + 512 bytes at M <= 64, the K-sliced path's partial
 * sums up to all of the scratch at M <= 16, the bf16 prefill path 2 * M * K
 * bytes). Every such call on one GPU shares
 * that scratch, which keeps the last call's contents (no kernel relies on it
 * starting at zero): calls that overlap in time on one GPU (other streams,
 * other contexts, other threads) race and must be serialized by the caller. */
#define DGM_NOALLOC_SCRATCH_BYTES (8u << 20)
int dgm_gemmNT_noalloc(dgm_gpu* g, int64_t bits, const float* w, const void* q,
                       const float* scale, const float* x, const float* bias, float* y,
                       int64_t M, int64_t N, int64_t K, int64_t qGroup);
/* No counterpart in the reference, whose buffers are all allocated at setup
 * (src/GPU.swift:31-88; its kernels never allocate). dgm_gemmNT's staging
 * buffers (activation pieces of the decode-shaped kernels, partial sums of the
 * K-sliced kernel, the bf16 copy of X of the prefill path) come from a
 * workspace of the context that is otherwise allocated by the first call that
 * needs it. dgm_gemmNT_workspace_bound returns bytes that cover every path a
 * dgm_gemmNT call of that shape can take, in either math mode (-1 for
 * negative sizes); dgm_gpu_reserve grows the workspace to at least `bytes`
 * now (DGM_ERR_UNSUPPORTED during a graph capture), so that later calls whose
 * bound it covers allocate nothing; dgm_gpu_workspace_bytes returns its size
 * (0 before anything was allocated). */
int64_t dgm_gemmNT_workspace_bound(int64_t M, int64_t N, int64_t K);
int dgm_gpu_reserve(dgm_gpu* g, int64_t bytes);
int64_t dgm_gpu_workspace_bytes(const dgm_gpu* g);
/* GPU.gemmDX (src/GPU.swift:245-260). */
int dgm_gemmDX(dgm_gpu* g, int64_t bits, const float* w, const void* q,
               const float* scale, const float* dy, float* dx,
               int64_t M, int64_t N, int64_t K, int64_t qGroup);
/* GPU.gemmDW (src/GPU.swift:262-266). */
int dgm_gemmDW(dgm_gpu* g, const float* dy, const float* x, float* dw,
               int64_t M, int64_t N, int64_t K);
/* GPU.gemmDWAcc (src/GPU.swift:268-272). */
int dgm_gemmDWAcc(dgm_gpu* g, const float* dy, const float* x, float* dw,
                  int64_t M, int64_t N, int64_t K);

/* GPU.gemmDW (accumulate = 0) or GPU.gemmDWAcc (accumulate != 0) followed by
 * GPU.gemmDX with the same dY: the pair the reference's backward issues back
 * to back for every linear (src/GPT.swift:374-376, 384-420). One launch when
 * the shapes allow (the dX and dW tiles run side by side), else the two
 * calls; either way dx and dw are bitwise what the two calls produce. */
int dgm_gemmBwd(dgm_gpu* g, int64_t bits, const float* w, const void* q, const float* scale,
                const float* dy, const float* x, float* dx, float* dw, int64_t M, int64_t N,
                int64_t K, int64_t qGroup, int accumulate);

/* ---- looped DiT block forward: the non-GEMM wrappers it calls -------------
 * Same names, buffer order and sizes as the Swift wrappers; fp32 buffers in
 * device memory. Layouts: activations [B,T,H,D] (rows of H*D), scores/probs
 * [B,H,T,T], RoPE tables [T,D]. */

/* GPU.rmsFwd (src/GPU.swift:364-367; rmsnorm_fwd, metal/kernels.metal:807-825):
 * y = x * rsqrt(mean(x^2) + eps) * weight per row; rstd[row] = that rsqrt
 * (rstd may be NULL). */
int dgm_rmsFwd(dgm_gpu* g, const float* x, float* y, float* rstd, const float* weight,
               int64_t rows, int64_t cols, float eps);
/* GPU.ropeFwd (src/GPU.swift:375-378; rope_fwd, metal/kernels.metal:871-889):
 * rotate-half RoPE; D must be even. */
int dgm_ropeFwd(dgm_gpu* g, const float* x, float* y, const float* cos_t, const float* sin_t,
                int64_t B, int64_t T, int64_t H, int64_t D);
/* GPU.repeatHeads (src/GPU.swift:407-410; repeat_heads, metal/kernels.metal:980-993):
 * dst[b,t,h,:] = src[b,t,:]. */
int dgm_repeatHeads(dgm_gpu* g, const float* src, float* dst, int64_t B, int64_t T, int64_t H,
                    int64_t D);
/* GPU.attnFwd (src/GPU.swift:302-310; attn_scores/attn_softmax/attn_av,
 * metal/kernels.metal:443-506), one fused kernel: scores = q.k / sqrt(D)
 * (masked to -1e30 above the diagonal when causal), probs = row softmax,
 * av = probs.v. Needs (2*T*D + 16*D + 16*T)*4 bytes <= 160 KiB of LDS. */
int dgm_attnFwd(dgm_gpu* g, const float* q, const float* k, const float* v, float* scores,
                float* probs, float* av, int64_t B, int64_t T, int64_t H, int64_t D, int causal);
/* GPU.swigluFwd (src/GPU.swift:385-387; swiglu_fwd, metal/kernels.metal:911-930):
 * y = gate * sigmoid(gate) * up. */
int dgm_swigluFwd(dgm_gpu* g, const float* gate, const float* up, float* y, int64_t n);
/* GPU.add (src/GPU.swift:211-213; add_f, metal/kernels.metal:419-427): y = a + b. */
int dgm_add(dgm_gpu* g, const float* a, const float* b, float* y, int64_t n);
/* GPU.mix (src/GPU.swift:393-396; mix_f, metal/kernels.metal:951-959): y = ca*a + cb*b. */
int dgm_mix(dgm_gpu* g, const float* a, const float* b, float* y, int64_t n, float ca, float cb);
/* GPU.copy (src/GPU.swift:398-400; copy_f, metal/kernels.metal:961-968): y = x. */
int dgm_copy(dgm_gpu* g, const float* x, float* y, int64_t n);

/* ropeTables (src/Macro.swift:509-530), host side: fills cos_t/sin_t, each
 * maxT*dim floats of HOST memory, with cos/sin(t * theta^(-2i/dim)) for
 * i < dim/2, repeated in both halves of each row. dim must be even. */
int dgm_ropeTables(int64_t maxT, int64_t dim, float theta, float* cos_t, float* sin_t);

/* The DiT block configuration the loop body reads (src/DiT.swift:9-41):
 * B sequences of T tokens, embd C = H*D, SwiGLU width F, one KV head of
 * width D repeated to H heads. bits 8 / 4 route every linear through the
 * group-quantized forward (group `group`); bits 32 uses the fp32 weights. */
typedef struct dgm_dit_cfg {
    int32_t B, T, C, F, H, D, loops, group, bits;
    float eps, mix;
    int32_t pad;
} dgm_dit_cfg;

/* One linear: fp32 weight w [N,K] (bits 32) or codes q + scales (bits 8/4). */
typedef struct dgm_dit_linear {
    const float* w;
    const void* q;
    const float* scale;
} dgm_dit_linear;

/* The block's parameters (src/DiT.swift:242-253): wq [C,C], wk/wv [D,C],
 * wo [C,C], wgate/wup [F,C], wdown [C,F]; RMSNorm weights of C floats. */
typedef struct dgm_dit_weights {
    dgm_dit_linear wq, wk, wv, wo, wgate, wup, wdown;
    const float *n1, *n1b, *n2, *n2b, *nf;
} dgm_dit_weights;

/* Floats of device workspace dgm_dit_forward needs for cfg (-1 for NULL). */
int64_t dgm_dit_workspace_floats(const dgm_dit_cfg* cfg);
/* The looped block forward (src/DiT.swift:520-550): x holds xs[0] [B*T, C] on
 * entry and xs[loops] on exit. cos_t/sin_t are device copies of
 * ropeTables(T, D, theta). ws: device workspace of at least
 * dgm_dit_workspace_floats(cfg) floats; on exit it holds the last loop's
 * intermediates (projections, scores and probs [B,H,T,T], attention output,
 * residual stream, SwiGLU input and output). When wq, wk, wv (and wgate,
 * wup) are laid out back to back in memory (codes and scales, or fp32
 * weights), each group runs as one GEMM. RoPE, the value-residual mix and the
 * KV-head broadcast are applied inside the attention kernel, and each
 * RMSNorm + residual chain is one row kernel; every element is computed as
 * the standalone wrappers compute it. Needs T and D multiples of 16 and
 * C <= 1024 (DGM_ERR_UNSUPPORTED otherwise); x, ws and the tables 16-byte
 * aligned. Enqueued on the context's
 * stream; graph-capturable (no allocation, no host sync). */
int dgm_dit_forward(dgm_gpu* g, const dgm_dit_cfg* cfg, const dgm_dit_weights* w,
                    const float* cos_t, const float* sin_t, float* x, float* ws,
                    int64_t ws_floats);

/* ---- looped DiT block backward (src/DiT.swift:558-626) ---------------------
 * The wrappers the backward loop calls, with the Swift names and buffer
 * order, then a forward that saves every loop's activations and the block
 * backward. */

/* GPU.rmsBwd (src/GPU.swift:369-373; rmsnorm_bwd_dx / rmsnorm_bwd_dw,
 * metal/kernels.metal:827-868): dx per row from the saved rstd, and
 * dweight[c] += sum over rows of dy*x*rstd (the weight is shared by every
 * loop). eps is accepted for the signature and unused, as in the reference. */
int dgm_rmsBwd(dgm_gpu* g, const float* x, const float* rstd, const float* weight, const float* dy,
               float* dx, float* dweight, int64_t rows, int64_t cols, float eps);
/* GPU.attnBwd (src/GPU.swift:312-322; attn_bwd_dv, attn_bwd_dp,
 * attn_softmax_bwd, attn_bwd_dq, attn_bwd_dk, metal/kernels.metal:508-612):
 * q, k, v, dout, dq, dk, dv [B,T,H,D]; probs, dprobs, dscores [B,H,T,T]. */
int dgm_attnBwd(dgm_gpu* g, const float* q, const float* k, const float* v, const float* probs,
                const float* dout, float* dq, float* dk, float* dv, float* dprobs, float* dscores,
                int64_t B, int64_t T, int64_t H, int64_t D);
/* GPU.ropeBwd (src/GPU.swift:380-383; rope_bwd, metal/kernels.metal:891-909). */
int dgm_ropeBwd(dgm_gpu* g, const float* dy, float* dx, const float* cos_t, const float* sin_t,
                int64_t B, int64_t T, int64_t H, int64_t D);
/* GPU.swigluBwd (src/GPU.swift:389-391; swiglu_bwd, metal/kernels.metal:932-949). */
int dgm_swigluBwd(dgm_gpu* g, const float* gate, const float* up, const float* dy, float* dgate,
                  float* dup, int64_t n);
/* GPU.sumHeads (src/GPU.swift:412-415; sum_heads, metal/kernels.metal:995-1010):
 * dst[b,t,:] = sum over h of src[b,t,h,:]. */
int dgm_sumHeads(dgm_gpu* g, const float* src, float* dst, int64_t B, int64_t T, int64_t H, int64_t D);
/* GPU.acc / GPU.accScale (src/GPU.swift:216-218, 402-405; acc_f, acc_scale_f,
 * metal/kernels.metal:429-436, 970-977): a += b, a += s*b. */
int dgm_acc(dgm_gpu* g, float* a, const float* b, int64_t n);
int dgm_accScale(dgm_gpu* g, float* a, const float* b, int64_t n, float s);

/* Gradients of the block's parameters, fp32, accumulated (+=): the seven
 * linears [N,K] as in dgm_dit_weights and the five RMSNorm weights [C]. */
typedef struct dgm_dit_grads {
    float *wq, *wk, *wv, *wo, *wgate, *wup, *wdown;
    float *n1, *n1b, *n2, *n2b, *nf;
} dgm_dit_grads;

/* Floats of the activation buffer dgm_dit_forward_train fills (-1 for NULL). */
int64_t dgm_dit_acts_floats(const dgm_dit_cfg* cfg);
/* Floats of workspace dgm_dit_backward needs (-1 for NULL). */
int64_t dgm_dit_backward_ws_floats(const dgm_dit_cfg* cfg);
/* The loop body of DiT.forward (src/DiT.swift:520-550) with every loop's
 * activations saved in acts (the reference's Acts): x holds xs[0] on entry
 * and xs[loops] on exit. Linears as in dgm_dit_forward (bits 32: fp32
 * weights; bits 8 / 4: codes + scales). */
int dgm_dit_forward_train(dgm_gpu* g, const dgm_dit_cfg* cfg, const dgm_dit_weights* w,
                          const float* cos_t, const float* sin_t, float* x, float* acts,
                          int64_t acts_floats);
/* The loop part of DiT.backward (src/DiT.swift:566-626) over the activations
 * of dgm_dit_forward_train: gx holds dL/dxs[loops] on entry and dL/dxs[0] on
 * exit; the parameter gradients are added into *grads. bits 32 runs dX on
 * the fp32 weights, as the reference does; bits 8 / 4 run it through the
 * dequantized codes (straight-through estimator) and dW into the fp32
 * gradients. ws: dgm_dit_backward_ws_floats(cfg) floats. */
int dgm_dit_backward(dgm_gpu* g, const dgm_dit_cfg* cfg, const dgm_dit_weights* w,
                     const dgm_dit_grads* grads, const float* cos_t, const float* sin_t,
                     const float* acts, int64_t acts_floats, float* gx, float* ws,
                     int64_t ws_floats);

/* ---- training step around the path: optimizer, re-quantize, embedding ----
 * GPT.step (src/GPT.swift:183-220) zeroes the grads, runs the backward, sums
 * the squared grads for clipping, scales them, applies AdamW to every master
 * weight and re-quantizes the quantized ones; the quantized GPT's token
 * embedding is the other consumer of the codes (src/GPT.swift:332-336,
 * 371-376, 425-429). Parameter blocks are the reference's (src/Params.swift). */

typedef struct dgm_AdamP {                     /* src/Params.swift:138-147      */
    uint32_t n;
    float lr, b1, b2, eps, wd, invBC1, invBC2;
} dgm_AdamP;                                   /* 32 bytes (src/GPU.swift:469)  */
typedef struct dgm_EmbP { uint32_t B, T, C, qGroup; } dgm_EmbP;       /* :78-83   */
typedef struct dgm_EmbBwdP { uint32_t B, T, C, V; } dgm_EmbBwdP;      /* :85-90   */
typedef struct dgm_PosP { uint32_t B, T, C, pad; } dgm_PosP;          /* :92-97   */
typedef struct dgm_BiasP { uint32_t M, N, pad0, pad1; } dgm_BiasP;    /* :46-51   */
typedef struct dgm_ReduceP { uint32_t n, slot, pad0, pad1; } dgm_ReduceP; /* :106-111 */
typedef struct dgm_ScaleP { uint32_t n; float s; uint32_t pad0, pad1; } dgm_ScaleP; /* :39-44 */
typedef struct dgm_UnaryP { uint32_t n, pad0, pad1, pad2; } dgm_UnaryP; /* :32-37  */

/* adamw (metal/kernels.metal:786-802), per element i < n:
 *   m = b1*m + (1-b1)*g;  v = b2*v + (1-b2)*g*g;
 *   w -= lr * ((m*invBC1) / (sqrt(v*invBC2) + eps) + wd*w)
 * each operation rounded to fp32 separately (no fused multiply-add). */
int dgm_adamw(dgm_gpu* g, float* w, const float* grad, float* m, float* v, const dgm_AdamP* p);
/* GPU.adam (src/GPU.swift:425-429). */
int dgm_adam(dgm_gpu* g, float* w, const float* grad, float* m, float* v, int64_t n,
             float lr, float b1, float b2, float eps, float wd, float invBC1, float invBC2);
/* GPU.adam followed by GPU.quantize of the same master (the quantized
 * parameters of src/GPT.swift:214-217 then quantizeAll, 441-447), in one pass
 * over the [rows, cols] master when cols % qGroup == 0 and qGroup is a power
 * of two in [8, 512]: w, m, v, q and scale come out bit-identical to the two
 * calls (which run instead for any other shape). No single reference
 * counterpart; it replaces that pair of dispatches. */
int dgm_adam_quantize(dgm_gpu* g, float* w, const float* grad, float* m, float* v, void* q,
                      float* scale, int64_t rows, int64_t cols, int64_t bits, int64_t qGroup,
                      float lr, float b1, float b2, float eps, float wd, float invBC1,
                      float invBC2);

/* reduce_sumsq (metal/kernels.metal:749-768): out[slot] = sum of x[i]^2,
 * i < n. The sum is taken in a fixed order of this library's own (per-block
 * partial sums over contiguous ranges, then a tree), so repeated calls give
 * identical bits; it agrees with the reference's 256-lane order to fp32
 * rounding, not bitwise. */
int dgm_reduce_sumsq(dgm_gpu* g, const float* x, float* out, const dgm_ReduceP* p);
/* GPU.reduceSumsq (src/GPU.swift:420-422). */
int dgm_reduceSumsq(dgm_gpu* g, const float* x, float* into, int64_t n, int64_t slot);
/* zero_f / scale_f (metal/kernels.metal:770-784); GPU.zero / GPU.scale
 * (src/GPU.swift:200-209). */
int dgm_zero_f(dgm_gpu* g, float* x, const dgm_UnaryP* p);
int dgm_scale_f(dgm_gpu* g, float* x, const dgm_ScaleP* p);
int dgm_zero(dgm_gpu* g, float* x, int64_t n);
int dgm_scale(dgm_gpu* g, float* x, int64_t n, float s);

/* embed_f32 / embed_i8 / embed_i4 (metal/kernels.metal:616-663):
 * y[bt, c] = wte[tok, c] + wpe[bt % T, c], with wte dequantized as
 * code * scale[tok, c / qGroup] for the quantized forms (rounded, then
 * added). tokens are uint32 ids < the table's rows (not checked). */
int dgm_embed_f32(dgm_gpu* g, const uint32_t* tokens, const float* wte, const float* wpe,
                  float* y, const dgm_EmbP* p);
int dgm_embed_i8(dgm_gpu* g, const uint32_t* tokens, const int8_t* wte, const float* scale,
                 const float* wpe, float* y, const dgm_EmbP* p);
int dgm_embed_i4(dgm_gpu* g, const uint32_t* tokens, const uint8_t* wte, const float* scale,
                 const float* wpe, float* y, const dgm_EmbP* p);
/* GPU.embed (src/GPU.swift:324-338): bits selects the kernel; wte is read
 * for bits 32, q and scale for bits 8 / 4. */
int dgm_embed(dgm_gpu* g, int64_t bits, const uint32_t* tokens, const float* wte, const void* q,
              const float* scale, const float* wpe, float* y, int64_t B, int64_t T, int64_t C,
              int64_t qGroup);
/* embed_bwd (metal/kernels.metal:665-682): dwe[v, c] += sum over bt with
 * tokens[bt] == v of dx[bt, c], summed in increasing bt (the reference's
 * order, so results are bitwise the reference's). Every row v < V is
 * rewritten. */
int dgm_embed_bwd(dgm_gpu* g, const uint32_t* tokens, const float* dx, float* dwe,
                  const dgm_EmbBwdP* p);
/* GPU.embedBwd (src/GPU.swift:340-344). */
int dgm_embedBwd(dgm_gpu* g, const uint32_t* tokens, const float* dx, float* dwe, int64_t B,
                 int64_t T, int64_t C, int64_t V);
/* pos_bwd (metal/kernels.metal:684-697): dwp[t, c] = sum over b (increasing)
 * of dx[b*T + t, c]; overwrites. */
int dgm_pos_bwd(dgm_gpu* g, const float* dx, float* dwp, const dgm_PosP* p);
/* GPU.posBwd (src/GPU.swift:346-350). */
int dgm_posBwd(dgm_gpu* g, const float* dx, float* dwp, int64_t B, int64_t T, int64_t C);
/* bias_grad (metal/kernels.metal:285-295): db[n] = sum over m (increasing) of
 * dY[m, n]; overwrites. */
int dgm_bias_grad(dgm_gpu* g, const float* dY, float* db, const dgm_BiasP* p);
/* GPU.biasGrad (src/GPU.swift:274-277). */
int dgm_biasGrad(dgm_gpu* g, const float* dy, float* db, int64_t M, int64_t N);

/* ---- checkpoints (host code, no context) ----------------------------------
 * The reference's checkpoint files: a little-endian header, then every
 * parameter's fp32 master in the model's creation order. These validate a
 * file image in host memory and describe each parameter; the caller uploads
 * the masters and re-quantizes the quantized ones (GPT.load calls
 * quantizeAll, src/GPT.swift:318-322). Return DGM_ERR_SHAPE for a wrong magic
 * or version, an invalid configuration, or a length that does not match the
 * model (the reference's preconditions). */
typedef struct dgm_tgmt_header {   /* GPT.save (src/GPT.swift:265-281) */
    uint32_t version, bits, vocab, block, layers, heads, embd, qGroup;
} dgm_tgmt_header;
typedef struct dgm_tdit_header {   /* DiT.save (src/DiT.swift:396-411) */
    uint32_t version, side, patch, names, loops, heads, kvHeads, embd, intermediate, freqDim,
        diffusionSteps;
    float lastAlpha, valueMix;      /* version 1 files carry no lastAlpha: 0.01 */
    uint32_t header_bytes;          /* where the first parameter starts       */
} dgm_tdit_header;
typedef struct dgm_param_info {
    char name[32];                  /* the reference's parameter name          */
    int64_t rows, cols;
    int32_t quantized, decay;       /* Param.quantized / Param.decay           */
    int64_t offset;                 /* byte offset of its fp32 data in the file */
} dgm_param_info;

/* GPT.load (src/GPT.swift:283-324): header, itos at *itos_offset (vocab
 * bytes), then 2 + 16*layers + 2 parameters (wte, wpe, per layer ln1.g ...
 * proj.b, ln_f.g, ln_f.b; src/GPT.swift:44-64, 118-131). */
int dgm_tgmt_parse(const void* data, int64_t len, dgm_tgmt_header* hdr, int64_t* itos_offset,
                   int64_t* nparams);
int dgm_tgmt_param(const dgm_tgmt_header* hdr, int64_t i, dgm_param_info* out);
/* DiT.load (src/DiT.swift:413-451): 17 parameters, wpatch ... wdown, n1 ... nf
 * (src/DiT.swift:233-250). */
int dgm_tdit_parse(const void* data, int64_t len, dgm_tdit_header* hdr, int64_t* nparams);
int dgm_tdit_param(const dgm_tdit_header* hdr, int64_t i, dgm_param_info* out);

/* ---- measurement ----------------------------------------------------------
 * No counterpart in the reference: the achievable HBM read rate of one
 * launch, for the bench's roofline. Reads `bytes` (a multiple of 1024) from
 * `src` (16-byte aligned) in contiguous shares over `workgroups` workgroups
 * (0: one per CU), mode 0 with 16-byte loads into registers, mode 1 with
 * 16-byte direct-to-LDS loads, and stores one word per workgroup to `sink`
 * (device memory of at least 4 * workgroups bytes). */
int dgm_probe_read(dgm_gpu* g, const void* src, int64_t bytes, int64_t mode, int64_t workgroups,
                   uint32_t* sink);
/* No counterpart in the reference: a wave-reduction VALU GEMV over int4 codes
 * (Y[M,N] = X[M,K] . dequant(Wq)^T, fp32 FMAs, no bias), the design the
 * library's MFMA decode kernels are measured against. M is 1 or 16; K and
 * qGroup are multiples of 32; Wq and X 16-byte aligned. */
int dgm_probe_gemv_valu(dgm_gpu* g, const uint8_t* Wq, const float* scale, const float* X, float* Y, int64_t M,
                        int64_t N, int64_t K, int64_t qGroup);

/* ---- test hook -------------------------------------------------------------
 * No counterpart in the reference: bounds every in-workgroup hand-over wait of
 * the decode kernels to `spins` rounds (0 restores the default), so that a
 * test can force a wait to give up and check that dgm_end reports it. The
 * kernels still run to their end; only their results are invalid. */
int dgm_debug_wait_limit(int64_t spins);

#ifdef __cplusplus
}
#endif

#endif /* DGM_QUANT_H */
