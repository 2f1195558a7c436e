/*
 * tmt_moe.h -- C ABI of the MI355X (gfx950) Mixture-of-Experts block.
 *
 * Drop-in for the MoE layer of TMT (reference tree, tmt-cuda/src/moe.cu):
 *   softmax router + top-k (ties -> lower expert index) + renormalised gates,
 *   Switch load-balancing aux loss and router z-loss with analytic gradients,
 *   SiLU experts, residual add (Y = beta*Y + MoE(X)).
 *
 * Two expert shapes:
 *   hidden == 0  reference experts: one linear W_e [d][d] per expert and
 *                SiLU applied in combine (moe.cu:142-158, 431-436).
 *   hidden  > 0  up/down experts: O = silu(X W_up^T) W_down^T with
 *                W_up [h][d] and W_down [d][h].
 * experts == 1 is the reference's dense path without a router
 * (moe.cu:397-403): Y = beta*Y + silu(X W_0^T) (hidden == 0).
 *
 * Layout: all matrices row-major, weights [out][in] like nn.Linear
 * (linalg.cu:1-8). bf16 values are raw uint16 bit patterns. Per-expert
 * weights are passed as host arrays of E device pointers, the reference's
 * `bf16** Wexp` convention (moe.cu:374).
 *
 * Widths: any d >= 1 and hidden >= 0, as TMT's validate_cfg
 * (config.h:46-52). When d and hidden are multiples of 64 the kernels read
 * the caller's tensors directly and every device pointer must be 16-byte
 * aligned. Other widths (TMT's own tests run dim 16 and 32) run on
 * zero-padded copies at the widths rounded up to 64, kept in the handle's
 * shared workspace: each call copies its operands in and its results out
 * (a few extra small kernels), and pointers need only their natural
 * alignment (2 bytes for bf16, 4 for fp32). Zero columns add exact zeros, so
 * the routing is the same as at the caller's width. The MXFP4 formats keep
 * d and hidden multiples of 64.
 *
 * Every function returns TMT_MOE_OK (0) or a negative error code and never
 * exits the process; tmt_moe_last_error() gives a thread-local message.
 * Forward and backward enqueue work on the given stream (hipStream_t passed
 * as void*; NULL = default stream) and never synchronise with the host.
 * A handle is single-layer state (the reference's MoeKeep + MoeWs,
 * moe.cu:294-328): forward saves routing for the following backward.
 * Calls on one handle must be ordered by the caller; different handles are
 * independent.
 */
#ifndef TMT_MOE_H
#define TMT_MOE_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
    TMT_MOE_OK = 0,
    TMT_MOE_EINVAL = -1,   /* bad argument, shape or alignment */
    TMT_MOE_ENOMEM = -2,   /* device allocation failed */
    TMT_MOE_EDEVICE = -3,  /* HIP runtime or launch error */
    TMT_MOE_ESTATE = -4    /* backward without a matching forward */
};

/* Expert weight formats (tmt_moe_desc::weight_format):
 *   BF16      bf16 weights, forward and backward;
 *   MXFP4     MXFP4 weights expanded to bf16 inside the GEMM, bf16
 *             activations: the products equal the fp32 products with the
 *             dequantised weights (forward only);
 *   MXFP4_MX  MXFP4 weights on the scaled MFMA, activations rounded to the
 *             sum of two MXFP6 (e2m3) terms per 32-element block (relative
 *             L2 error of the block output about 1e-3), about twice the MFMA
 *             rate of the bf16 products (forward only);
 *   MXFP4_MX_PLANES  the same arithmetic with the weight codes already in the
 *             kernels' K-plane layout (tmt_moe_mxfp4_planes), which spares
 *             each forward the copy into it. */
enum {
    TMT_MOE_WEIGHTS_BF16 = 0,
    TMT_MOE_WEIGHTS_MXFP4 = 1,
    TMT_MOE_WEIGHTS_MXFP4_MX = 2,
    TMT_MOE_WEIGHTS_MXFP4_MX_PLANES = 3
};

typedef struct tmt_moe_desc {
    int32_t max_tokens;     /* T_max: largest T a call may pass */
    int32_t d;              /* model width, >= 1 (TMT's config.h:46-52) */
    int32_t experts;        /* E, 1..64 */
    int32_t topk;           /* K, 1..min(E, 8) */
    int32_t hidden;         /* h >= 1, or 0 for reference experts */
    int32_t weight_format;  /* TMT_MOE_WEIGHTS_* */
} tmt_moe_desc;

typedef struct tmt_moe tmt_moe;

/* Replaces moe_keep_alloc + moe_ws_alloc (moe.cu:330-362): one device arena
 * sized from the descriptor; no allocation happens after this call. */
int tmt_moe_create(const tmt_moe_desc* desc, tmt_moe** out);
/* Replaces moe_keep_free + moe_ws_free (moe.cu:342-348, 363-370). */
int tmt_moe_destroy(tmt_moe* moe);
/* Arena bytes tmt_moe_create would allocate for this descriptor
 * (per_layer + shared of tmt_moe_workspace_sizes). */
int tmt_moe_workspace_size(const tmt_moe_desc* desc, size_t* bytes);

/*
 * The two parts of a handle's device memory (moe.cu:294-328):
 *   per_layer  state kept from forward to backward (the reference's MoeKeep:
 *              routing, offsets, permutation, expert activations, the
 *              LayerNorm output and row statistics);
 *   shared     buffers used only inside one call (the reference's MoeWs:
 *              router block tables, split-K partials and every backward
 *              operand), which layers that run one after another can share.
 * Either pointer may be NULL.
 */
int tmt_moe_workspace_sizes(const tmt_moe_desc* desc, size_t* per_layer, size_t* shared);

/*
 * Replaces moe_keep_alloc over a moe_ws_alloc'd workspace (moe.cu:330-362,
 * model.cu:252-254): the handle allocates only its per_layer part and uses
 * `workspace` (device memory, 256-byte aligned, at least the shared size of
 * tmt_moe_workspace_sizes for this descriptor) for the rest. Handles that
 * share a workspace must not run concurrently: order their calls on one
 * stream (or synchronise between streams), as the reference's layers run
 * one after another. The workspace must outlive every handle using it.
 */
int tmt_moe_create_shared(const tmt_moe_desc* desc, void* workspace, size_t workspace_bytes,
                          tmt_moe** out);

/*
 * Replaces moe_forward (moe.cu:374-466).
 *   X [T][d] bf16, Wr [E][d] bf16 (ignored when E == 1),
 *   logit_bias [E] fp32 device pointer or NULL (added to the router logits;
 *   NULL gives the reference's bias-free router, moe.cu:10-38),
 *   W_up[E]  -> [h][d] bf16   (hidden > 0)  or W_e [d][d] (hidden == 0),
 *   W_down[E]-> [d][h] bf16   (hidden > 0; NULL allowed when hidden == 0),
 *   Y [T][d] bf16 is read-modify-write: Y = beta*Y + MoE(X).
 * Unlike the reference there is no host synchronisation: counts, offsets
 * and the expert tile table stay on the device. The reference's returned
 * aux value and k.zloss are read with tmt_moe_read_stats.
 */
int tmt_moe_forward(tmt_moe* moe, void* stream, int32_t T, const uint16_t* X,
                    const uint16_t* Wr, const float* logit_bias,
                    const uint16_t* const* W_up, const uint16_t* const* W_down,
                    uint16_t* Y, float beta);

/*
 * MXFP4 variant of tmt_moe_forward for weight_format TMT_MOE_WEIGHTS_MXFP4,
 * TMT_MOE_WEIGHTS_MXFP4_MX or TMT_MOE_WEIGHTS_MXFP4_MX_PLANES
 * (no reference counterpart: the reference has no FP4 path). OCP MX format:
 * e2m1 values in blocks of 32 along the reduction dimension sharing one e8m0
 * scale 2^(s-127). Per expert e:
 *   W_up[e]        packed codes [h][d/2] bytes, low nibble = even column
 *   W_up_scale[e]  scales [d/32][h] bytes (block-major: the scales of one
 *                  K block are contiguous over the output rows)
 *   W_down[e]      [d][h/2] bytes,  W_down_scale[e]  [h/32][d] bytes.
 * With MXFP4, activations stay bf16 and the weights are expanded to bf16
 * (exactly) inside the GEMM, so the result matches the fp32 product with
 * dequantised weights. With MXFP4_MX, the block input and the SiLU output
 * are rounded to two MXFP6 terms and both expert GEMMs run on the scaled
 * FP6 x FP4 MFMA. Forward only: backward needs bf16 master weights.
 * With MXFP4_MX_PLANES, W_up[e] and W_down[e] hold the codes in K planes as
 * tmt_moe_mxfp4_planes writes them; the scales keep the layout above.
 */
int tmt_moe_forward_mxfp4(tmt_moe* moe, void* stream, int32_t T,
                          const uint16_t* X, const uint16_t* Wr,
                          const float* logit_bias,
                          const uint8_t* const* W_up, const uint8_t* const* W_up_scale,
                          const uint8_t* const* W_down, const uint8_t* const* W_down_scale,
                          uint16_t* Y, float beta);

/*
 * MXFP4 weight codes [N][K/2] (the layout above: N output rows, K reduction
 * columns, low nibble = even column) to K planes of 64 columns,
 * [K/64][N][32] bytes: plane p holds the 32 code bytes of columns 64p ..
 * 64p + 63 of every row, rows in order. No counterpart in the reference (it
 * has no FP4 path); for callers of TMT_MOE_WEIGHTS_MXFP4_MX_PLANES, who pack
 * each expert matrix once (W_up[e]: N = h, K = d; W_down[e]: N = d, K = h)
 * instead of every forward doing it. N and K multiples of 64; codes and
 * planes 16-byte aligned device buffers of N * K / 2 bytes; enqueued on
 * `stream` on the current device.
 */
int tmt_moe_mxfp4_planes(void* stream, const uint8_t* codes, int32_t N, int32_t K, uint8_t* planes);

/*
 * Replaces moe_backward (moe.cu:479-545) for the loss
 *   L = <dY, Y> + aux_coef * aux + z_coef * z
 * (aux_coef / z_coef already divided by the layer count, model.cu:677).
 * X is the forward input (the reference keeps a copy in MoeKeep::H,
 * moe.cu:396; here the caller passes it again). Outputs are overwritten:
 *   dX [T][d] bf16, dWr [E][d] fp32 (may be NULL when E == 1; when E == 1
 *   and non-NULL, its d floats are zeroed, as moe.cu:486-487 does),
 *   dW_up[E] -> [h][d] fp32 (or [d][d] when hidden == 0),
 *   dW_down[E] -> [d][h] fp32 (hidden > 0).
 * Experts that received no tokens get all-zero gradients (the reference
 * leaves them untouched, moe.cu:534-535).
 */
int tmt_moe_backward(tmt_moe* moe, void* stream, const uint16_t* dY,
                     const uint16_t* X, const uint16_t* Wr,
                     const uint16_t* const* W_up, const uint16_t* const* W_down,
                     float aux_coef, float z_coef, uint16_t* dX, float* dWr,
                     float* const* dW_up, float* const* dW_down);

/*
 * LayerNorm in front of the block, in one call: replaces the recurrent
 * block's layernorm_fwd + moe_forward pair (model.cu:509-514; norm.cu:8-50,
 * 96-100):
 *   H = LayerNorm(S; ln_gamma, ln_beta)  (eps 1e-5, biased variance),
 *   Y = beta*Y + MoE(H)                  (as tmt_moe_forward).
 * S [T][d] bf16; ln_gamma, ln_beta [d] fp32 device pointers. H, the row
 * mean and 1/std stay in the handle's arena for tmt_moe_backward_ln.
 * Row statistics follow one fixed summation order, so H is bit-identical
 * run to run (the reference's block-tree order is not reproducible).
 * bf16 weights only.
 */
int tmt_moe_forward_ln(tmt_moe* moe, void* stream, int32_t T, const uint16_t* S,
                       const float* ln_gamma, const float* ln_beta,
                       const uint16_t* Wr, const float* logit_bias,
                       const uint16_t* const* W_up, const uint16_t* const* W_down,
                       uint16_t* Y, float beta);

/*
 * Backward of tmt_moe_forward_ln: replaces moe_backward + layernorm_bwd
 * (model.cu:674-680; norm.cu:53-106). Must follow tmt_moe_forward_ln on the
 * same handle; S is the forward's LayerNorm input, passed again. The gradient
 * at H stays in the arena (bf16, like the reference's m.dH). Outputs are
 * overwritten:
 *   dS [T][d] bf16, dGamma, dBeta [d] fp32 (summed over rows in a fixed
 *   order; the reference zeroes them and adds with atomics, norm.cu:102-105),
 *   dWr, dW_up, dW_down as tmt_moe_backward.
 */
int tmt_moe_backward_ln(tmt_moe* moe, void* stream, const uint16_t* dY,
                        const uint16_t* S, const float* ln_gamma,
                        const uint16_t* Wr, const uint16_t* const* W_up,
                        const uint16_t* const* W_down, float aux_coef, float z_coef,
                        uint16_t* dS, float* dGamma, float* dBeta, float* dWr,
                        float* const* dW_up, float* const* dW_down);

/*
 * Replaces the host read of the router statistics (moe.cu:448-465 and
 * moe_aux_from, moe.cu:470-475). Waits for `stream`, then writes the Switch
 * aux loss E*sum_e(mean_p_e*frac_e), the z-loss mean(lse^2) and the
 * per-expert token counts [E] (the reference's hcnt, capi.cu:131-136) of the
 * last forward. Any output pointer may be NULL.
 */
int tmt_moe_read_stats(tmt_moe* moe, void* stream, float* aux, float* z,
                       int32_t* counts);

/* Device address of the last forward's statistics: float {aux, z} followed
 * by E int32 counts. Lets a caller batch the read of many layers, like the
 * reference's deferred k.stat slot (moe.cu:311-314, model.cu:542-549). */
int tmt_moe_stats_device_ptr(tmt_moe* moe, const void** ptr);

/*
 * Parity/debug: waits for `stream` and copies the last forward's routing to
 * host memory. Any pointer may be NULL. Shapes: logits, probs [T][E] fp32;
 * idx [T][K] int32; gate [T][K] fp32 (renormalised weights);
 * offsets [E+1] int32 (expert segment starts); perm [T*K] int32 (token of
 * each slot, stable: ascending token inside a segment); slot_of [T][K].
 */
int tmt_moe_read_routing(tmt_moe* moe, void* stream, float* logits,
                         float* probs, int32_t* idx, float* gate,
                         int32_t* offsets, int32_t* perm, int32_t* slot_of);

/*
 * Standalone LayerNorm, no handle: replaces layernorm_fwd / layernorm_bwd
 * (norm.cu:96-106), e.g. for the LayerNorm in front of the reference's MLA
 * block (model.cu:521-522, 667-669). Same kernels and summation order as
 * tmt_moe_forward_ln / tmt_moe_backward_ln (d > 2048 path).
 *   forward:  H = LayerNorm(S; gamma, beta) (eps 1e-5), mean / rstd [T] out.
 *   backward: from the bf16 gradient dH at H: dS [T][d] bf16, dGamma, dBeta
 *             [d] fp32 (overwritten, fixed-order sums over rows).
 * The backward needs `workspace` of at least tmt_moe_layernorm_workspace_size
 * bytes (device memory, 256-byte aligned); no call allocates. Any d >= 1
 * (rows whose width is not a multiple of 8 are read and written element by
 * element, in the same summation order); pointers 16-byte aligned. Calls
 * that share a workspace must be ordered by the caller.
 */
int tmt_moe_layernorm_workspace_size(int32_t T, int32_t d, size_t* bytes);
int tmt_moe_layernorm_forward(void* stream, int32_t T, int32_t d, const uint16_t* S,
                              const float* gamma, const float* beta, uint16_t* H,
                              float* mean, float* rstd);
int tmt_moe_layernorm_backward(void* stream, int32_t T, int32_t d, const uint16_t* S,
                               const uint16_t* dH, const float* gamma, const float* mean,
                               const float* rstd, uint16_t* dS, float* dGamma, float* dBeta,
                               void* workspace, size_t workspace_bytes);

/*
 * tmt_moe_layernorm_backward without the workspace argument, for callers
 * that cannot allocate device memory (code under HIP graph capture, tight
 * serving loops, harnesses that forbid hipMalloc). No reference counterpart.
 * The scratch is a 4 MiB device array inside the library (one per GPU, held
 * until the process ends): shapes whose workspace
 * (tmt_moe_layernorm_workspace_size) exceeds 4 MiB are rejected with
 * TMT_MOE_EINVAL, e.g. T = 32768 at d = 1024 uses 0.53 MiB. No call
 * allocates. Every call on one GPU uses that GPU's same scratch: calls that
 * overlap on one GPU (different streams, or threads, without ordering) race.
 * The first call on a device looks the scratch's address up and keeps it for
 * the process: make that first call outside a graph capture, and do not use
 * the entry point after hipDeviceReset. Later calls may be captured (the
 * launches are plain kernels, no memset nodes). Same results, bit for bit,
 * as tmt_moe_layernorm_backward.
 */
int tmt_moe_layernorm_backward_noalloc(void* stream, int32_t T, int32_t d, const uint16_t* S,
                                       const uint16_t* dH, const float* gamma, const float* mean,
                                       const float* rstd, uint16_t* dS, float* dGamma, float* dBeta);

/*
 * Parity/debug: waits for `stream` and copies what the last
 * tmt_moe_forward_ln kept: H [T][d] bf16, mean and rstd [T] fp32 (the
 * reference's Ly.mean / Ly.rstd, model.cu:510-511). Any pointer may be NULL.
 */
int tmt_moe_read_norm(tmt_moe* moe, void* stream, uint16_t* H, float* mean,
                      float* rstd);

/*
 * Per-kernel timing, the counterpart of the reference's TMT_PROFILE phase
 * timers (moe.cu:380-394, 459-464), but with HIP events on the call's stream
 * instead of device-wide synchronisation. While enabled, every kernel launch
 * of forward/backward is bracketed by two events. tmt_moe_read_profile waits
 * for the recorded events and returns, per phase, the summed milliseconds and
 * the number of launches since the last reset (arrays of TMT_MOE_NPHASES).
 */
enum {
    TMT_MOE_PH_ROUTER = 0, TMT_MOE_PH_SCAN, TMT_MOE_PH_PERMUTE, TMT_MOE_PH_GEMM_UP,
    TMT_MOE_PH_GEMM_DOWN, TMT_MOE_PH_COMBINE, TMT_MOE_PH_COMBINE_BWD, TMT_MOE_PH_GEMM_DACT,
    TMT_MOE_PH_GEMM_DW_DOWN, TMT_MOE_PH_GEMM_DW_UP, TMT_MOE_PH_GEMM_DX, TMT_MOE_PH_ROUTER_DW,
    TMT_MOE_PH_SCATTER, TMT_MOE_PH_NORM, TMT_MOE_PH_NORM_BWD, TMT_MOE_NPHASES
};
int tmt_moe_set_profiling(tmt_moe* moe, int enable);
int tmt_moe_read_profile(tmt_moe* moe, float* ms, int32_t* launches, int reset);
const char* tmt_moe_phase_name(int phase);

/*
 * Multi-tensor AdamW with global-norm gradient clipping over fp32 master
 * weights, moments and gradients, e.g. the block's router and expert
 * parameters with the fp32 gradients tmt_moe_backward writes. Replaces the
 * reference's multi-tensor optimizer (MTParams + mt_sumsq_kernel +
 * mt_adam_kernel + mt_zero_kernel, adam.cu:37-96; table built once,
 * model.cu:436-454; optimizer_step, model.cu:716-729).
 *
 * tmt_moe_adamw_create copies the parameter list into a device chunk table
 * (chunks of 8192 elements) and allocates all state; no later call
 * allocates. Every pointer must be 16-byte aligned device memory; `work`
 * may be NULL. flags: TMT_MOE_ADAMW_IN_NORM (the gradient counts in the
 * clipping norm), TMT_MOE_ADAMW_UPDATE (the parameter is updated).
 *
 * tmt_moe_adamw_step enqueues, with `step` the 1-based update count
 * (bias corrections 1 - beta^step, as the reference's powf(b, step + 1) with
 * its 0-based step):
 *   s = sum of grad^2 over IN_NORM parameters (double, one fixed order);
 *   if s is finite, for every UPDATE parameter, elementwise:
 *     g = grad * scale, scale = clip > 0 ? min(1, clip / max(sqrt(s), 1e-12)) : 1
 *     m = b1 m + (1 - b1) g;  v = b2 v + (1 - b2) g g
 *     w = w - lr ((m / bc1) / (sqrt(v / bc2) + eps) + wd w);  work = bf16(w)
 *   else nothing is updated (the reference refuses the step).
 * tmt_moe_adamw_read_sumsq waits for `stream` and returns s of the last step
 * (the reference's one host read per step); the caller refuses non-finite.
 * tmt_moe_adamw_zero_grads sets every gradient to zero (model.cu:592).
 * Calls on one optimizer must be ordered by the caller.
 */
enum { TMT_MOE_ADAMW_IN_NORM = 1, TMT_MOE_ADAMW_UPDATE = 2 };
typedef struct tmt_moe_adamw_param {
    float* master;     /* [n] fp32 master weights */
    float* m;          /* [n] first moment */
    float* v;          /* [n] second moment */
    float* grad;       /* [n] fp32 gradient */
    uint16_t* work;    /* [n] bf16 working copy, or NULL */
    int64_t n;
    int32_t flags;
} tmt_moe_adamw_param;
typedef struct tmt_moe_adamw tmt_moe_adamw;
int tmt_moe_adamw_create(const tmt_moe_adamw_param* params, int32_t count, tmt_moe_adamw** out);
int tmt_moe_adamw_destroy(tmt_moe_adamw* opt);
int tmt_moe_adamw_step(tmt_moe_adamw* opt, void* stream, float clip, float lr, float beta1,
                       float beta2, float eps, float weight_decay, int32_t step);
int tmt_moe_adamw_read_sumsq(tmt_moe_adamw* opt, void* stream, double* sumsq);
int tmt_moe_adamw_zero_grads(tmt_moe_adamw* opt, void* stream);
/* Number of chunks (workgroups per launch) of an optimizer. */
int tmt_moe_adamw_chunks(tmt_moe_adamw* opt, int32_t* chunks);

/* out[i] = bf16(in[i]) (round to nearest even) for n fp32 values: the bf16
 * work copy of fp32 master weights, replacing copy_bf16_kernel
 * (tmt-cuda/src/model.cu:54; used after initialisation and loads,
 * model.cu:219, checkpoint.h:149). */
int tmt_moe_f32_to_bf16(void* stream, const float* in, uint16_t* out, int64_t n);

/* Thread-local message of the last failing call on this thread. */
const char* tmt_moe_last_error(void);

#ifdef __cplusplus
}
#endif
#endif
