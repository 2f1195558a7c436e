/*
 * moe_oracle.h -- CPU restatement of TMT's Mixture-of-Experts block.
 *
 * TEST INFRASTRUCTURE ONLY. This library is the parity checker for the HIP
 * implementation. Only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg may load it. The product path never calls into it.
 *
 * Every routine restates reference semantics and cites the reference lines
 * (paths relative to the reference tree):
 *   router + softmax + top-k + renorm  tmt-cuda/src/moe.cu:72-95 (topk_kernel,
 *                                      the general-E rule), moe.cu:10-68
 *   counts / dispatch                  tmt-cuda/src/moe.cu:97-115, 409-424
 *   experts + combine                  tmt-cuda/src/moe.cu:142-158, 431-436
 *   aux / z-loss                       tmt-cuda/src/moe.cu:257-278, 453-465
 *   backward                           tmt-cuda/src/moe.cu:160-249, 477-545
 *   numerics (silu, silu')             tmt-cuda/src/common.h:15-24
 *   GEMM layouts ([out,in], fp32 acc)  tmt-cuda/src/linalg.cu:1-41
 *   LayerNorm                          tmt-cuda/src/norm.cu:8-106
 *   multi-tensor AdamW                 tmt-cuda/src/adam.cu:37-96, model.cu:716-729
 *
 * Conventions shared with the HIP library (include/tmt_moe.h):
 *   bf16 values are raw uint16 bit patterns; fp32 accumulation everywhere.
 *   Wr [E][d]; W_up[e] [h][d]; W_down[e] [d][h]; in h == 0 mode the expert
 *   is the reference's single linear W_e [d][d] passed as W_up[e].
 *   Router logits use the canonical summation order documented at
 *   orc_router_logit(); selection is on logits, strict '>' over ascending
 *   expert index (ties go to the lower index).
 *   The permutation is stable: inside an expert segment slots follow
 *   ascending token index.
 *
 * All entry points return 0 on success and a negative value on bad
 * arguments. Threading is deterministic: results are bit-identical for any
 * thread count.
 */
#ifndef TMT_MOE_ORACLE_H
#define TMT_MOE_ORACLE_H
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct orc_dims {
    int32_t T;        /* tokens */
    int32_t d;        /* model width */
    int32_t E;        /* experts (1 = dense path, no router) */
    int32_t K;        /* top-k */
    int32_t h;        /* expert hidden; 0 = reference single-linear experts */
    int32_t threads;  /* worker threads (<= 0: hardware concurrency) */
} orc_dims;

/* Round-to-nearest-even fp32 -> bf16 and exact bf16 -> fp32. */
void orc_f32_to_bf16(const float* in, uint16_t* out, int64_t n);
void orc_bf16_to_f32(const uint16_t* in, float* out, int64_t n);

/* One canonical router logit (see the definition in moe_oracle.cpp). */
float orc_router_logit(const uint16_t* x, const uint16_t* w, int32_t d);

/* Router: logits/probs [T][E], idx/w [T][K], lse [T]. bias may be NULL. */
int orc_router(const orc_dims* dm, const uint16_t* X, const uint16_t* Wr,
               const float* bias, float* logits, float* probs, int32_t* idx,
               float* w, float* lse);

/* Dispatch: counts [E], offsets [E+1], perm [T*K], slot_of [T][K]. */
int orc_dispatch(const orc_dims* dm, const int32_t* idx, int32_t* counts,
                 int32_t* offsets, int32_t* perm, int32_t* slot_of);

/* Switch aux loss and z-loss from probs, counts and lse. */
int orc_aux_z(const orc_dims* dm, const float* probs, const int32_t* counts,
              const float* lse, float* aux, float* z);

/*
 * Full forward (fp32). Y_out[T][d] = beta*Y_in + sum_j w_j * expert_j(x).
 * Y_in may be NULL when beta == 0. Routing outputs may be NULL.
 * W_up / W_down are arrays of E host pointers; W_down is ignored if h == 0.
 */
int orc_forward(const orc_dims* dm, const uint16_t* X, const uint16_t* Wr,
                const float* bias, const uint16_t* const* W_up,
                const uint16_t* const* W_down, const uint16_t* Y_in,
                float beta, float* Y_out, float* logits, float* probs,
                int32_t* idx, float* w, int32_t* counts, int32_t* offsets,
                int32_t* perm, int32_t* slot_of, float* aux, float* z);

/*
 * Full backward (fp32) for loss = sum(dY * Y) + aux_coef*aux + z_coef*z.
 * Recomputes the forward internally. dW_up / dW_down are arrays of E host
 * pointers (fp32, overwritten; zero for idle experts). dWr may be NULL for
 * E == 1. dW_down is ignored if h == 0.
 */
int orc_backward(const orc_dims* dm, const uint16_t* X, const uint16_t* Wr,
                 const float* bias, const uint16_t* const* W_up,
                 const uint16_t* const* W_down, const uint16_t* dY,
                 float aux_coef, float z_coef, float* dX, float* dWr,
                 float* const* dW_up, float* const* dW_down);

/*
 * fp64 twin for finite differences on tiny shapes. Inputs are doubles so a
 * test can perturb any of them. Routing is recomputed in fp64 (plain order).
 * loss = sum(dY*Y) + aux_coef*aux + z_coef*z, where frac_e = cnt_e/(T*K) is
 * treated as a constant exactly as the reference's router_bwd_kernel does.
 * Gradients are written when the output pointers are non-NULL.
 */
int orc_loss_f64(const orc_dims* dm, const double* X, const double* Wr,
                 const double* bias, const double* W_up, const double* W_down,
                 const double* dY, double aux_coef, double z_coef,
                 double* loss, double* dX, double* dWr, double* dW_up,
                 double* dW_down, int32_t* idx_out);

/* Router regularizer gradient on given logits (restates test_router). */
int orc_router_bwd(const orc_dims* dm, const float* logits, const int32_t* idx,
                   const float* s, const int32_t* counts, float aux_coef,
                   float z_coef, float* dlogits);

/* MXFP4: quantise fp32 rows of length n (multiple of 32) to packed e2m1
 * nibbles (low nibble = even element) plus one e8m0 scale per 32 values,
 * and the exact inverse. */
int orc_mxfp4_quantize(const float* in, int64_t rows, int64_t n,
                       uint8_t* packed, uint8_t* scales);
int orc_mxfp4_dequantize(const uint8_t* packed, const uint8_t* scales,
                         int64_t rows, int64_t n, float* out);

/* LayerNorm that precedes the MoE in TMT (tmt-cuda/src/norm.cu:8-106).
 * Forward: H [T][d] bf16, mean/rstd [T]; statistics in the canonical order
 * documented at ln_row_stats() (the GPU kernel's order). Backward from the
 * fp32 gradient dH: dS [T][d], dgamma/dbeta [d] (fp32, overwritten). */
int orc_layernorm_fwd(int32_t T, int32_t d, const uint16_t* S, const float* gamma,
                      const float* beta, uint16_t* H, float* mean, float* rstd);
int orc_layernorm_bwd(int32_t T, int32_t d, const uint16_t* S, const float* dH,
                      const float* gamma, const float* mean, const float* rstd,
                      float* dS, float* dgamma, float* dbeta);

/* Multi-tensor AdamW with global-norm clipping (tmt-cuda/src/adam.cu:37-96,
 * optimizer_step tmt-cuda/src/model.cu:716-729), one step in place over
 * `count` parameters; flags bit 0: gradient in the norm, bit 1: updated.
 * `step` is the 1-based update count (bias corrections 1 - b^step). The
 * squared gradient norm is summed in the canonical order documented at
 * adamw_chunk_sum() and orc_adamw_step() (the GPU kernels' order) and
 * returned in *sumsq; a non-finite norm leaves every parameter unchanged. */
int orc_adamw_step(int32_t count, float* const* master, float* const* m, float* const* v,
                   const float* const* grad, uint16_t* const* work, const int64_t* n,
                   const int32_t* flags, float clip, float lr, float b1, float b2, float eps,
                   float wd, int32_t step, double* sumsq);

#ifdef __cplusplus
}
#endif
#endif
