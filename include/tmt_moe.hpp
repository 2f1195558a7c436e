/*
 * tmt_moe.hpp -- C++17 host interface with the reference's MoE operator
 * signatures, layered on the C ABI of tmt_moe.h.
 *
 * The reference's MoE layer is a set of header-inline C++ functions compiled
 * into each program (tmt-cuda/src/moe.cu:294-545). This header offers the
 * same names with the same argument meaning, so a call site such as
 * tmt-cuda/src/model.cu:512-514 or :676-677 compiles against it unchanged:
 *
 *   MoeKeep / MoeWs                     moe.cu:294-328
 *   moe_keep_alloc / moe_keep_free      moe.cu:330-348
 *   moe_ws_alloc / moe_ws_free          moe.cu:349-370
 *   moe_forward                         moe.cu:372-466
 *   moe_aux_from                        moe.cu:468-475
 *   moe_backward                        moe.cu:477-545
 *   layernorm_fwd / layernorm_bwd       norm.cu:96-106
 *   moe_expert_counts                   capi.cu:131-136 (tmt_model_expert_counts)
 *   moe_router_balance                  train_main.cu:232-248 (router balance log)
 *
 * Behaviour kept from the reference:
 *   - experts are single d x d linears with SiLU inside combine (hidden = 0);
 *     moe_keep_alloc's extra `hidden` argument selects the up/SiLU/down
 *     expert, whose forward/backward take a second weight table;
 *   - moe_forward saves a copy of X in MoeKeep::H for the backward
 *     (moe.cu:396), returns the Switch aux loss and sets MoeKeep::zloss, or,
 *     when MoeKeep::stat is set, only copies the statistics there and returns
 *     0 (moe.cu:448-452); moe_aux_from then yields aux and zloss;
 *   - MoeKeep::hcnt holds the per-expert token counts after the statistics
 *     were read (read by tmt_model_expert_counts, capi.cu:131-136);
 *   - moe_backward overwrites dX, dWrouter and dWexp (linalg.cu:32-41 with
 *     beta 0); experts without tokens get zero gradients;
 *   - errors print a message and exit(1), as CUDA_CHECK does
 *     (common.h:26-33); callers that want status codes use tmt_moe.h.
 * Work goes to MoeKeep::stream (default: the null stream, the reference's
 * default stream). Unlike the reference there is no host synchronisation
 * inside moe_forward when MoeKeep::stat is set, and none in moe_backward.
 * MoeWs is, as in the reference, one set of transient buffers shared by all
 * layers (model.cu:104, 254): moe_ws_alloc sizes it from the layer shape
 * (tmt_moe_workspace_sizes' shared part), and each layer's handle is created
 * on its first moe_forward over the MoeWs passed there
 * (tmt_moe_create_shared). Layers sharing one MoeWs must run one after
 * another, as the reference's do. A MoeKeep used with an MoeWs that was
 * never allocated gets a private workspace.
 */
#pragma once

#include <hip/hip_runtime_api.h>

#include <cstdint>
#include <cstdio>
#include <cstdlib>

#include "tmt_moe.h"

struct MoeKeep {
    float zloss = 0;
    float* stat = nullptr;          // optional caller-owned device slot (>= 2 floats: aux, z)
    const float* bias = nullptr;    // optional [E] fp32 logit bias (not in the reference)
    hipStream_t stream = nullptr;
    uint16_t* H = nullptr;          // [N][D] bf16 copy of the forward input
    int32_t hcnt[64] = {0};         // tokens per expert (after the statistics were read)
    int N = 0, E = 0, K = 0, D = 0, hidden = 0, max_N = 0;
    tmt_moe* handle = nullptr;  // created by the first moe_forward
};
struct MoeWs {
    void* ptr = nullptr;  // device workspace shared by the layers
    size_t bytes = 0;
};

namespace tmt_moe_detail {
[[noreturn]] inline void die(const char* where, const char* what) {
    std::printf("%s: %s\n", where, what);
    std::fflush(stdout);
    std::exit(1);
}
inline void check(int rc, const char* where) {
    if (rc != TMT_MOE_OK) die(where, tmt_moe_last_error());
}
inline void check_hip(hipError_t e, const char* where) {
    if (e != hipSuccess) die(where, hipGetErrorString(e));
}
template <class B>
inline const uint16_t* bits(const B* p) {
    static_assert(sizeof(B) == 2, "bf16 element type expected");
    return reinterpret_cast<const uint16_t*>(p);
}
template <class B>
inline uint16_t* bits(B* p) {
    static_assert(sizeof(B) == 2, "bf16 element type expected");
    return reinterpret_cast<uint16_t*>(p);
}
template <class B>
inline const uint16_t* const* table(B* const* p) {
    static_assert(sizeof(B) == 2, "bf16 element type expected");
    return reinterpret_cast<const uint16_t* const*>(p);
}

inline tmt_moe_desc keep_desc(const MoeKeep& k) {
    tmt_moe_desc desc{};
    desc.max_tokens = k.max_N > 0 ? k.max_N : 1;
    desc.d = k.D;
    desc.experts = k.E;
    desc.topk = k.K;
    desc.hidden = k.hidden;
    desc.weight_format = TMT_MOE_WEIGHTS_BF16;
    return desc;
}

// Copy the input for the backward, run the forward, deliver the statistics.
inline float forward(const uint16_t* X, const uint16_t* Wr, const uint16_t* const* Wup,
                     const uint16_t* const* Wdown, uint16_t* Y, MoeKeep& k, MoeWs& w, int N, int E,
                     int K, int D, float beta) {
    const char* where = "moe_forward";
    if (k.E == 0) die(where, "moe_keep_alloc was not called");
    if (!k.handle) {
        const tmt_moe_desc desc = keep_desc(k);
        check(w.ptr ? tmt_moe_create_shared(&desc, w.ptr, w.bytes, &k.handle) : tmt_moe_create(&desc, &k.handle),
              where);
    }
    if (E != k.E || K != k.K || D != k.D) die(where, "E, K or D differ from moe_keep_alloc");
    if (N < 0 || N > k.max_N) die(where, "N exceeds the moe_keep_alloc size");
    k.N = N;
    if (N > 0) check_hip(hipMemcpyAsync(k.H, X, (size_t)N * D * 2, hipMemcpyDeviceToDevice, k.stream), where);
    check(tmt_moe_forward(k.handle, k.stream, N, X, Wr, k.bias, Wup, Wdown, Y, beta), where);
    if (E == 1) return 0.f;  // dense path: no router statistics (moe.cu:397-403)
    if (k.stat) {            // deferred: the owner reads all layers at once
        const void* st = nullptr;
        check(tmt_moe_stats_device_ptr(k.handle, &st), where);
        check_hip(hipMemcpyAsync(k.stat, st, 2 * sizeof(float), hipMemcpyDeviceToDevice, k.stream), where);
        k.zloss = 0;
        return 0.f;
    }
    float aux = 0, z = 0;
    check(tmt_moe_read_stats(k.handle, k.stream, &aux, &z, k.hcnt), where);
    k.zloss = z;
    return aux;
}

inline void backward(const uint16_t* dY, const uint16_t* const* Wup, const uint16_t* const* Wdown,
                     const uint16_t* Wr, float* dWr, float* const* dWup, float* const* dWdown,
                     uint16_t* dX, MoeKeep& k, float aux, float zcoef) {
    const char* where = "moe_backward";
    if (!k.handle) die(where, "no moe_forward ran on this layer");
    // With E == 1 the library zeroes dWr, as the reference does (moe.cu:487).
    check(tmt_moe_backward(k.handle, k.stream, dY, k.H, Wr, Wup, Wdown, aux, zcoef, dX, dWr, dWup,
                           dWdown), where);
}
}  // namespace tmt_moe_detail

/* moe.cu:330-341. N is the largest token count a forward will see. The
 * shape is checked here; the device state is created by the first
 * moe_forward, over the MoeWs it is given. */
inline void moe_keep_alloc(MoeKeep& k, int N, int E, int K, int D, int hidden = 0) {
    k.E = E; k.K = K; k.D = D; k.hidden = hidden; k.max_N = N;
    const tmt_moe_desc desc = tmt_moe_detail::keep_desc(k);
    size_t layer = 0, shared = 0;
    tmt_moe_detail::check(tmt_moe_workspace_sizes(&desc, &layer, &shared), "moe_keep_alloc");
    if (N > 0)
        tmt_moe_detail::check_hip(hipMalloc((void**)&k.H, (size_t)N * D * 2), "moe_keep_alloc");
}

/* moe.cu:342-348 */
inline void moe_keep_free(MoeKeep& k) {
    if (k.handle) tmt_moe_destroy(k.handle);
    if (k.H) (void)hipFree(k.H);
    k = MoeKeep();
}

/* moe.cu:349-362: the transient buffers every layer of this shape shares
 * (hidden selects the up/down expert, as in moe_keep_alloc). */
inline void moe_ws_alloc(MoeWs& w, int N, int E, int K, int D, int hidden = 0) {
    tmt_moe_desc desc{};
    desc.max_tokens = N > 0 ? N : 1;
    desc.d = D;
    desc.experts = E;
    desc.topk = K;
    desc.hidden = hidden;
    desc.weight_format = TMT_MOE_WEIGHTS_BF16;
    size_t layer = 0, shared = 0;
    tmt_moe_detail::check(tmt_moe_workspace_sizes(&desc, &layer, &shared), "moe_ws_alloc");
    tmt_moe_detail::check_hip(hipMalloc(&w.ptr, shared), "moe_ws_alloc");
    w.bytes = shared;
}

/* moe.cu:363-370. Free the layers' MoeKeep first. */
inline void moe_ws_free(MoeWs& w) {
    if (w.ptr) (void)hipFree(w.ptr);
    w = MoeWs();
}

/* moe.cu:372-466: Y = beta*Y + MoE(X) with the reference's single-linear
 * experts Wexp[e] [D][D] (hidden == 0). Returns the Switch aux loss. */
template <class B>
inline float moe_forward(const B* X, const B* Wrouter, B** Wexp, B* Y, MoeKeep& k, MoeWs& w,
                         int N, int E, int K, int D, float beta = 0.0f) {
    if (k.hidden != 0) tmt_moe_detail::die("moe_forward", "hidden > 0 needs the W_down table");
    using namespace tmt_moe_detail;
    return forward(bits(X), bits(Wrouter), table(Wexp), nullptr, bits(Y), k, w, N, E, K, D, beta);
}

/* Up/SiLU/down experts (hidden > 0): W_up[e] [hidden][D], W_down[e] [D][hidden]. */
template <class B>
inline float moe_forward(const B* X, const B* Wrouter, B** W_up, B** W_down, B* Y, MoeKeep& k,
                         MoeWs& w, int N, int E, int K, int D, float beta = 0.0f) {
    if (k.hidden == 0) tmt_moe_detail::die("moe_forward", "hidden == 0 takes one weight table");
    using namespace tmt_moe_detail;
    return forward(bits(X), bits(Wrouter), table(W_up), table(W_down), bits(Y), k, w, N, E, K, D, beta);
}

/* moe.cu:468-475: aux from the statistics moe_forward copied to k.stat
 * (hsum = the host copy of that slot); sets k.zloss and k.hcnt. */
inline float moe_aux_from(MoeKeep& k, const float* hsum) {
    if (!k.handle) tmt_moe_detail::die("moe_aux_from", "no moe_forward ran on this layer");
    k.zloss = hsum[1];
    tmt_moe_detail::check(tmt_moe_read_stats(k.handle, k.stream, nullptr, nullptr, k.hcnt),
                          "moe_aux_from");
    return hsum[0];
}

/* moe.cu:477-545: dX [N][D] bf16, dWrouter [E][D] fp32, dWexp[e] [D][D] fp32,
 * all overwritten; aux / zcoef are the loss coefficients (already / L). */
template <class B>
inline void moe_backward(const B* dY, B** Wexp, const B* Wrouter, float* dWrouter, float** dWexp,
                         B* dX, MoeKeep& k, MoeWs&, float aux = 0.f, float zcoef = 0.f) {
    if (k.hidden != 0) tmt_moe_detail::die("moe_backward", "hidden > 0 needs the W_down tables");
    using namespace tmt_moe_detail;
    backward(bits(dY), table(Wexp), nullptr, bits(Wrouter), dWrouter, dWexp, nullptr, bits(dX), k,
             aux, zcoef);
}

namespace tmt_moe_detail {
// Per-device workspace of layernorm_bwd, grown on demand and kept for the
// process (like the reference's lazily created cuBLAS handle, util.h:23-31;
// not thread-safe, as the reference's layer is not).
inline void* ln_workspace(size_t bytes) {
    static void* ws[64] = {};
    static size_t cap[64] = {};
    int dev = 0;
    check_hip(hipGetDevice(&dev), "layernorm_bwd");
    if (dev < 0 || dev >= 64) die("layernorm_bwd", "device index out of range");
    if (cap[dev] < bytes) {
        if (ws[dev]) {
            check_hip(hipDeviceSynchronize(), "layernorm_bwd");
            check_hip(hipFree(ws[dev]), "layernorm_bwd");
        }
        ws[dev] = nullptr;
        check_hip(hipMalloc(&ws[dev], bytes), "layernorm_bwd");
        cap[dev] = bytes;
    }
    return ws[dev];
}
}  // namespace tmt_moe_detail

/* norm.cu:96-100: Y = LayerNorm(X; gamma, beta), eps 1e-5; mean / rstd [N]
 * saved for the backward. On the null stream, like the reference. */
template <class B>
inline void layernorm_fwd(const B* X, const float* gamma, const float* beta, B* Y, float* mean,
                          float* rstd, int N, int D) {
    using namespace tmt_moe_detail;
    check(tmt_moe_layernorm_forward(nullptr, N, D, bits(X), gamma, beta, bits(Y), mean, rstd),
          "layernorm_fwd");
}

/* norm.cu:102-106: dX [N][D] bf16 from the bf16 gradient dY; dGamma and
 * dBeta [D] are overwritten (the reference zeroes them, then accumulates). */
template <class B>
inline void layernorm_bwd(const B* X, const B* dY, const float* gamma, const float* mean,
                          const float* rstd, B* dX, float* dGamma, float* dBeta, int N, int D) {
    using namespace tmt_moe_detail;
    size_t bytes = 0;
    check(tmt_moe_layernorm_workspace_size(N, D, &bytes), "layernorm_bwd");
    check(tmt_moe_layernorm_backward(nullptr, N, D, bits(X), bits(dY), gamma, mean, rstd, bits(dX),
                                     dGamma, dBeta, ln_workspace(bytes), bytes),
          "layernorm_bwd");
}

/* Up/SiLU/down experts: dW_up[e] [hidden][D], dW_down[e] [D][hidden] fp32. */
template <class B>
inline void moe_backward(const B* dY, B** W_up, B** W_down, const B* Wrouter, float* dWrouter,
                         float** dW_up, float** dW_down, B* dX, MoeKeep& k, MoeWs&,
                         float aux = 0.f, float zcoef = 0.f) {
    if (k.hidden == 0) tmt_moe_detail::die("moe_backward", "hidden == 0 takes one weight table");
    using namespace tmt_moe_detail;
    backward(bits(dY), table(W_up), table(W_down), bits(Wrouter), dWrouter, dW_up, dW_down,
             bits(dX), k, aux, zcoef);
}

/* capi.cu:131-136 (tmt_model_expert_counts): the token count of every expert
 * of every layer in the last forward, out[l * E + e], from each layer's
 * MoeKeep::hcnt (filled when that layer's statistics were read). */
inline void moe_expert_counts(const MoeKeep* layers, int L, int64_t* out) {
    for (int l = 0; l < L; ++l)
        for (int e = 0; e < layers[l].E; ++e) out[(int64_t)l * layers[l].E + e] = layers[l].hcnt[e];
}

/* train_main.cu:232-248: the router-balance line over token counts `use`
 * [L][E] accumulated across steps. Each (layer, expert) pair's share is
 * use / total * L * E (1.0 = uniform); min starts at 1 and max at 0, as in
 * the reference, and a pair with share < 0.01 counts as dead. */
struct MoeBalance {
    double min = 1, max = 0;
    long dead = 0;
    int pairs = 0;
};
inline MoeBalance moe_router_balance(const int64_t* use, int L, int E) {
    MoeBalance b;
    b.pairs = L * E;
    long double tot = 0;
    for (int i = 0; i < L * E; ++i) tot += (long double)use[i];
    for (int i = 0; i < L * E; ++i) {
        const double s = tot > 0 ? (double)((long double)use[i] / tot * L * E) : 0.0;
        if (s < b.min) b.min = s;
        if (s > b.max) b.max = s;
        if (s < 0.01) ++b.dead;
    }
    return b;
}
