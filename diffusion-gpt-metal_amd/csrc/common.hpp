// Internal helpers shared by the HIP translation units of libdgm_amd.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>
#include <cstdio>
#include <cstring>

#include "../../include/dgm_quant.h"
#include "dw_tile.hpp"

// Context behind the opaque dgm_gpu handle (mirrors class GPU, src/GPU.swift:91-198).
struct dgm_gpu {
    int device = 0;
    int num_cus = 256;
    hipStream_t own_stream = nullptr;
    hipStream_t stream = nullptr;
    bool begun = false;
    int math = DGM_MATH_FP32;
    int first_err = DGM_OK;           // first error since begin()
    char last_kernel[64] = {0};
    char err_msg[320] = {0};
    // Grow-only device workspace for staging (the decode kernels' activation
    // pieces, sum-of-squares partials). Owned by the context. A grown
    // workspace keeps its predecessors (at most kMaxRetired, each at most half
    // the next) until dgm_gpu_destroy, since queued work and captured graphs
    // may still use them.
    static constexpr int kMaxRetired = 48;
    void* ws = nullptr;
    size_t ws_bytes = 0;
    void* retired[kMaxRetired] = {};
    int n_retired = 0;
    // The static device scratch of the allocation-free entry point (its
    // address on this context's device, resolved in dgm_gpu_create), and
    // whether the current call draws its workspace from it instead.
    void* scratch = nullptr;
    bool use_scratch = false;
    // Streams the context was set to (dgm_gpu_set_stream), synchronized by
    // dgm_gpu_destroy; and whether a kernel with bounded in-workgroup waits
    // ran since the last dgm_end (which then checks their give-up flag).
    static constexpr int kMaxStreams = 16;
    hipStream_t streams[kMaxStreams] = {};
    int n_streams = 0;
    bool many_streams = false;   // more than kMaxStreams: destroy waits for the device
    bool spin_waits = false;
};

namespace dgm {

// Records an error on the context (keeps the first one of the region) and
// returns the code so call sites can `return fail(...)`.
int fail(dgm_gpu* g, int code, const char* fmt, ...) __attribute__((format(printf, 3, 4)));

// Marks `name` as the last dispatched kernel (GPU.lastKernel) and checks that
// a begin()/end() region is open.
int enter(dgm_gpu* g, const char* name);

// Checks hipGetLastError() after a launch.
int check_launch(dgm_gpu* g, const char* name);

// Ensures the context workspace holds at least `bytes`; returns nullptr on
// failure (error recorded): allocation failure, or growth needed while the
// context's stream is capturing a graph.
void* workspace(dgm_gpu* g, size_t bytes);
// The status a caller returns when workspace() gave nullptr.
int ws_error(dgm_gpu* g);
// After a synchronize: records an error on g if a decode kernel gave up a
// bounded in-workgroup wait since the last check (gemm_decode.hip), and
// clears the device's flag.
void decode_wait_check(dgm_gpu* g);
// Bytes of the static device scratch behind dgm_gemmNT_noalloc.
constexpr size_t kScratchBytes = size_t(8) << 20;

constexpr int64_t kMaxIndex = (int64_t(1) << 31) - 1;

// Where the DiT block's training forward stores one loop's activations (the
// reference's Acts, src/DiT.swift:260-300): x, ln1 and its rstd, q / k / v
// as the attention consumed them ([B*T, C], k and v repeated to every head;
// dit_forward_loops stores only the KV head, columns 0 .. D-1, which is all
// dit_attn_bwd_loop reads),
// probs, av, attn, rstd of rms(attn), mid, ln2 and its rstd, gate, up, sw,
// mlp, rstd of rms(mlp), pre, rstd of rms(pre).
struct DitSaves {
    float *x, *ln1, *r1, *q, *k, *v, *probs, *av, *attn, *r1b, *mid, *ln2, *r2, *gate, *up, *sw, *mlp, *r2b, *pre,
        *rf;
};
// The training forward on the fused loop-body kernels (dit.hip), storing the
// activations of every loop into saves[0 .. loops-1]. Returns kNotFused
// (recording nothing) when the weights or sizes do not fit the fused kernels,
// so the caller runs the kernel-per-wrapper sequence instead.
constexpr int kNotFused = -1;
int64_t dit_train_scratch_floats(const dgm_dit_cfg* c);
int dit_forward_train_fused(dgm_gpu* g, const dgm_dit_cfg* c, const dgm_dit_weights* w, const float* cosv,
                            const float* sinv, float* x, const DitSaves* saves, float* scratch,
                            int64_t scratch_floats);
// The three-launch loop body (dit_loop.hip): whether the config is one of its
// built shapes (int8 / int4, group 32, C % 64 == 0, F % 128 == 0),
// whether the weights also fit it (linears back to back, aligned), and the
// floats of its wdown slabs ([F / 128][B*T][C]).
bool dit_loop_shape_ok(const dgm_dit_cfg* c);
bool dit_loop_ok(const dgm_dit_cfg* c, const dgm_dit_weights* w);
int64_t dit_loop_part_floats(const dgm_dit_cfg* c);
// Buffers of the loops: the wdown slabs and loop 0's v [B*T, D]; for the
// inference run also (the training run keeps these in its saves) q [B*T, C],
// k and v [B*T, D], two [B*T, C] buffers that alternate as mid, ln2
// [B*T, C], and the last loop's probs (may be null).
struct DitLoopBufs {
    float* part;
    float* vfirst;
    float *q, *k, *v;
    float* mid[2];
    float* ln2;
    float* probs_last;
};
// Runs the loops on x in place; saves (null for inference) as for
// dit_forward_train_fused. Needs dit_loop_ok.
int dit_forward_loops(dgm_gpu* g, const dgm_dit_cfg* c, const dgm_dit_weights* w, const float* cosv,
                      const float* sinv, float* x, const DitLoopBufs& buf, const DitSaves* saves);
// The attention backward of one loop of a built shape (dit_loop.hip), from
// the saved q, k, v ([B*T, C], k and v repeated to every head), probs and av
// and dL/d(av): the gradients of q before RoPE, of k before RoPE and of v
// before the value mix (summed over the heads), and dfirst updated (loop 0:
// first = true; fresh = true when dfirst holds nothing yet, which the first
// loop the backward runs then writes instead of adding to). Returns
// kNotFused, launching nothing, unless dit_attn_bwd_loop_ok holds for the
// activation and workspace buffers (16-byte aligned pieces).
bool dit_attn_bwd_loop_ok(const dgm_dit_cfg* c, const float* acts, const float* ws);
// dw (may be null): the 32 x 16 tiles of one linear's dW, run by extra
// workgroups of the same launch beside the attention backward (they read
// none of its outputs).
int dit_attn_bwd_loop(dgm_gpu* g, const dgm_dit_cfg* c, const float* q, const float* k, const float* v,
                      const float* probs, const float* o, const float* dout, const float* cosv, const float* sinv,
                      float* dq, int ldq, float* dk, float* dv, int ldkv, float* dfirst, bool first, bool fresh,
                      const dgm_dw::DwTileArgs* dw = nullptr);
// True when `next`'s weights (fp32 for bits 32, else codes and scales)
// start where `first`'s `rows` x K end, so the two act as one [2 rows, K]
// linear.
bool dit_linear_follows(const dgm_dit_linear& first, const dgm_dit_linear& next, int64_t rows, int64_t K, int bits,
                        int G);

// SwiGLU backward of one element (metal/kernels.metal:911-918 for the
// sign-split logistic, 932-949 for the derivative), fp contraction off:
// dgate = silu'(z) * u * g, dup = silu(z) * g.
__device__ inline void swiglu_bwd_value(float z, float u, float g, float& dgate, float& dup) {
#pragma clang fp contract(off)
    float s;
    if (z >= 0.0f) {
        const float e = expf(-z);
        s = 1.0f / (1.0f + e);
    } else {
        const float e = expf(z);
        s = e / (1.0f + e);
    }
    const float silu = z * s;
    const float siluP = s * (1.0f + z * (1.0f - s));
    dgate = siluP * u * g;
    dup = silu * g;
}

// The same with the logistic's exponential as the hardware 2^x of x log2 e
// (e^-|z| for both signs, no branch; within a few ulp of expf), as the DiT
// loop kernels' forward SwiGLU computes it.
__device__ inline void swiglu_bwd_value_hw(float z, float u, float g, float& dgate, float& dup) {
#pragma clang fp contract(off)
    const float e = __builtin_amdgcn_exp2f(-fabsf(z) * 1.44269504088896341f);
    const float s = z >= 0.0f ? 1.0f / (1.0f + e) : e / (1.0f + e);
    const float silu = z * s;
    const float siluP = s * (1.0f + z * (1.0f - s));
    dgate = siluP * u * g;
    dup = silu * g;
}

// gemmBwd (dW += dY^T X, dX = dY W) of a linear whose input was
// SwiGLU(gate, up) [M, K], with the SwiGLU backward applied to dX in the same
// launch: dgu gets [M, 2K] rows [dgate | dup]. Returns kNotFused, having
// launched nothing, when the shapes do not fit the one-launch pair.
int gemm_bwd_swiglu(dgm_gpu* g, int bits, const float* w, const void* q, const float* scale, const float* dy,
                    const float* x, const float* gate, const float* up, float* dgu, float* dw, int64_t M, int64_t N,
                    int64_t K, int64_t qGroup);

// The STE backward of a quantized linear with dX on bf16 MFMA (gemm_f32.hip):
// wt_prep writes the codes (int8, also for int4) and scales of up to 4
// linears transposed, codesT [K][N] and scalesT [K/G][N], one launch;
// gemm_bwd_fold then runs dX from them (the group scale folded into dY,
// which is split into three bf16 pieces) beside the fp32 dW tiles
// (dW += or = dY^T X; dW null: the dX tiles alone), with the SwiGLU
// backward on dX when sg_gate is set.
// gemm_bwd_fold returns kNotFused, launching nothing, unless bwd_fold_ok
// holds and the buffers are aligned (dY and scalesT 16 bytes, codesT 8).
int wt_prep(dgm_gpu* g, int bits, int nlin, const void* const* W, const float* const* S, const int* N, const int* K,
            int G, int8_t* const* codesT, float* const* scalesT);
bool bwd_fold_ok(int M, int N, int K, int G);
int gemm_bwd_fold(dgm_gpu* g, const int8_t* codesT, const float* scalesT, const float* dY, const float* X, float* dX,
                  float* dW, int M, int N, int K, int G, bool accumulate, const float* sg_gate, const float* sg_up);

inline bool aligned(const void* p, size_t a) {
    return (reinterpret_cast<uintptr_t>(p) & (a - 1)) == 0;
}

inline unsigned ceil_div(int64_t a, int64_t b) { return unsigned((a + b - 1) / b); }

}  // namespace dgm

#define DGM_LAUNCH_CHECK(g, name)                         \
    do {                                                  \
        int _rc = ::dgm::check_launch((g), (name));       \
        if (_rc != DGM_OK) return _rc;                    \
    } while (0)
